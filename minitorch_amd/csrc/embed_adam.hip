// Embedding gather / deterministic scatter-add, and multi-tensor Adam (fp32).
//
// Embedding.forward is Tensor.__getitem__ with an index array
// (layers.py:102-104 -> tensor.py:374-387); its backward is
// np.add.at(grad, idx, out.grad) (tensor.py:382).  Repeated ids must add up:
// here one workgroup owns one table row and adds the matching token rows in
// token order, so the result is deterministic (no atomics).
//
// Adam.step (optim.py:37-59) over every parameter tensor in one launch: the
// caller passes a device table with one entry per tensor.  The arithmetic
// follows the reference's float32 expression order:
//   m = b1*m + (1-b1)*g;  v = b2*v + (1-b2)*(g*g)
//   p -= (lr * (m / (1-b1^t))) / (sqrt(v / (1-b2^t)) + eps)
#include "mtx_common.h"

#include <cmath>

namespace mtx {
namespace {

__global__ __launch_bounds__(256) void embed_gather_kernel(const float* __restrict__ w, int64_t ldw,
                                                           const int64_t* __restrict__ idx,
                                                           float* __restrict__ out, int64_t ldo, int64_t n, int C,
                                                           int64_t V) {
  const int64_t total = n * C;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / C;
    const int c = (int)(e % C);
    int64_t r = idx[i];
    r = r < 0 ? 0 : (r >= V ? V - 1 : r);  // ids are validated on the host
    out[i * ldo + c] = w[r * ldw + c];
  }
}

// dW[v, c] (+)= sum over tokens i with idx[i] == v of g[i, c], in token order
__global__ __launch_bounds__(256) void embed_scatter_kernel(const int64_t* __restrict__ idx,
                                                            const float* __restrict__ g, int64_t ldg,
                                                            float* __restrict__ dw, int64_t lddw, int64_t n, int C,
                                                            int accumulate) {
  __shared__ int64_t ids[256];
  const int64_t v = blockIdx.x;
  const int c = blockIdx.y * 256 + threadIdx.x;
  float acc = 0.f;
  for (int64_t base = 0; base < n; base += 256) {
    const int64_t i = base + threadIdx.x;
    __syncthreads();
    ids[threadIdx.x] = i < n ? idx[i] : -1;
    __syncthreads();
    const int cnt = (int)min<int64_t>(256, n - base);
    if (c < C) {
      for (int j = 0; j < cnt; ++j)
        if (ids[j] == v) acc += g[(base + j) * ldg + c];
    }
  }
  if (c < C) {
    float* p = dw + v * lddw + c;
    *p = accumulate ? *p + acc : acc;
  }
}

// out[i, v] = (idx[i] == v), row-major (n, V)
__global__ __launch_bounds__(256) void onehot_kernel(const int64_t* __restrict__ idx, int64_t n, int64_t V,
                                                     float* __restrict__ out) {
  const int64_t total = n * V;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / V, v = e % V;
    out[e] = idx[i] == v ? 1.0f : 0.0f;
  }
}

struct AdamEntry {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  int64_t block0;  // first block of this tensor
};

// Elements one 256-thread block of the multi-tensor kernels covers: 8 per
// thread, as two float4 accesses per array (the launch count of blocks stays
// in the thousands for a GPT's ~10M parameters, and each block locates its
// tensor once).
constexpr int kAdamChunk = 2048;

// The table entry whose blocks include this one: the last entry with
// block0 <= blockIdx.x (binary search; block0 ascends with the entry).
__device__ __forceinline__ const AdamEntry& adam_owner(const AdamEntry* __restrict__ tab, int ntab) {
  const int64_t bx = blockIdx.x;
  int lo = 0, hi = ntab - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tab[mid].block0 <= bx) lo = mid; else hi = mid - 1;
  }
  return tab[lo];
}

struct AdamCoef {
  float lr, b1, b2, c1, c2, bc1, bc2, eps, wd;
};

// one element's update; bc1, bc2 = the step's bias corrections 1 - b^t.
// Every product and sum is rounded on its own (no fused multiply-add), as
// NumPy evaluates the reference's float32 expressions, so the update is
// bit-identical to it for the same gradient.
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, const AdamCoef& k) {
#pragma clang fp contract(off)
  if (k.wd != 0.f) g = g + k.wd * p;
  m = k.b1 * m + k.c1 * g;
  v = k.b2 * v + k.c2 * (g * g);
  const float mh = m / k.bc1;
  const float vh = v / k.bc2;
  p = p - (k.lr * mh) / (sqrtf(vh) + k.eps);
}

__device__ __forceinline__ void adam_update(const AdamEntry* __restrict__ tab, int ntab, const AdamCoef& k) {
  const AdamEntry e = adam_owner(tab, ntab);
  const int64_t base = ((int64_t)blockIdx.x - e.block0) * kAdamChunk;
  const bool vec = ((reinterpret_cast<uintptr_t>(e.p) | reinterpret_cast<uintptr_t>(e.g) |
                     reinterpret_cast<uintptr_t>(e.m) | reinterpret_cast<uintptr_t>(e.v)) & 15) == 0;
#pragma unroll
  for (int j = 0; j < kAdamChunk / 1024; ++j) {
    const int64_t i = base + j * 1024 + threadIdx.x * 4;
    if (vec && i + 4 <= e.n) {
      float4 p = *reinterpret_cast<const float4*>(e.p + i);
      const float4 g = *reinterpret_cast<const float4*>(e.g + i);
      float4 m = *reinterpret_cast<const float4*>(e.m + i);
      float4 v = *reinterpret_cast<const float4*>(e.v + i);
      adam_elem(p.x, g.x, m.x, v.x, k);
      adam_elem(p.y, g.y, m.y, v.y, k);
      adam_elem(p.z, g.z, m.z, v.z, k);
      adam_elem(p.w, g.w, m.w, v.w, k);
      *reinterpret_cast<float4*>(e.m + i) = m;
      *reinterpret_cast<float4*>(e.v + i) = v;
      *reinterpret_cast<float4*>(e.p + i) = p;
    } else {
      for (int64_t q = i; q < i + 4 && q < e.n; ++q) {
        float p = e.p[q], m = e.m[q], v = e.v[q];
        adam_elem(p, e.g[q], m, v, k);
        e.m[q] = m;
        e.v[q] = v;
        e.p[q] = p;
      }
    }
  }
}

__global__ __launch_bounds__(256) void adam_kernel(const AdamEntry* __restrict__ tab, int ntab, AdamCoef k) {
  adam_update(tab, ntab, k);
}

// Graph-replayable Adam: the step count lives in device memory (incremented
// by the one-thread kernel below, launched just before the update), and the
// bias corrections come from a table the host fills with the same float32
// values mtx_adam_f32 computes, entry (t - 1) % len for step t.
__global__ void adam_count_kernel(int* __restrict__ step) { step[0] += 1; }

__global__ __launch_bounds__(256) void adam_dev_kernel(const AdamEntry* __restrict__ tab, int ntab, AdamCoef k,
                                                       const int* __restrict__ step, const float* __restrict__ bc,
                                                       int bc_len) {
  const int j = (step[0] - 1) % bc_len;
  k.bc1 = bc[2 * j];
  k.bc2 = bc[2 * j + 1];
  adam_update(tab, ntab, k);
}

// Zero every tensor's gradient in one launch (the capturable optimizer's
// zero_grad): same table and block layout as the update.
__global__ __launch_bounds__(256) void zero_grads_kernel(const AdamEntry* __restrict__ tab, int ntab) {
  const AdamEntry e = adam_owner(tab, ntab);
  float* g = const_cast<float*>(e.g);
  const int64_t base = ((int64_t)blockIdx.x - e.block0) * kAdamChunk;
  const bool vec = (reinterpret_cast<uintptr_t>(g) & 15) == 0;
#pragma unroll
  for (int j = 0; j < kAdamChunk / 1024; ++j) {
    const int64_t i = base + j * 1024 + threadIdx.x * 4;
    if (vec && i + 4 <= e.n) {
      *reinterpret_cast<float4*>(g + i) = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      for (int64_t q = i; q < i + 4 && q < e.n; ++q) g[q] = 0.f;
    }
  }
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_zero_grads_f32(const void* table, int ntensors, int64_t total_blocks, void* stream) {
  MTX_CHECK_ARG(table && ntensors >= 1, "zero_grads: empty table");
  MTX_CHECK_SHAPE(total_blocks >= 0 && total_blocks < (1LL << 31), "zero_grads: bad block count");
  if (total_blocks == 0) return MTX_OK;
  hipLaunchKernelGGL(zero_grads_kernel, dim3((unsigned)total_blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const AdamEntry*>(table), ntensors);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_adam_bias_table(double beta1, double beta2, int first_step, int len, float* out) {
  MTX_CHECK_ARG(out != nullptr && len >= 1 && first_step >= 1, "adam_bias_table: bad argument");
  for (int s = first_step; s < first_step + len; ++s) {
    const int j = (s - 1) % len;
    out[2 * j] = (float)(1.0 - std::pow(beta1, (double)s));
    out[2 * j + 1] = (float)(1.0 - std::pow(beta2, (double)s));
  }
  return MTX_OK;
}

extern "C" int mtx_adam_dev_f32(const void* table, int ntensors, int64_t total_blocks, double lr, double beta1,
                                double beta2, double eps, double weight_decay, int* step, const float* bias_table,
                                int table_len, void* stream) {
  MTX_CHECK_ARG(table && ntensors >= 1 && step && bias_table && table_len >= 1, "adam_dev: null or empty argument");
  MTX_CHECK_SHAPE(total_blocks >= 0 && total_blocks < (1LL << 31), "adam_dev: bad block count");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(adam_count_kernel, dim3(1), dim3(1), 0, st, step);
  MTX_LAUNCHED();
  if (total_blocks == 0) return MTX_OK;
  const AdamCoef k{(float)lr, (float)beta1, (float)beta2, (float)(1.0 - beta1), (float)(1.0 - beta2), 1.f, 1.f,
                   (float)eps, (float)weight_decay};
  hipLaunchKernelGGL(adam_dev_kernel, dim3((unsigned)total_blocks), dim3(256), 0, st,
                     static_cast<const AdamEntry*>(table), ntensors, k, step, bias_table, table_len);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_embedding_fwd_f32(const float* weight, int64_t ldw, int64_t V, const int64_t* idx, int64_t n,
                                     float* out, int64_t ldo, int C, void* stream) {
  MTX_CHECK_ARG(weight && idx && out, "embedding: null pointer");
  MTX_CHECK_SHAPE(n >= 0 && C >= 1 && V >= 1 && ldw >= C && ldo >= C, "embedding: bad shape");
  if (n == 0) return MTX_OK;
  const int blocks = (int)std::min<int64_t>((n * C + 255) / 256, 16384);
  hipLaunchKernelGGL(embed_gather_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), weight, ldw,
                     idx, out, ldo, n, C, V);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_embedding_bwd_f32(const int64_t* idx, int64_t n, const float* grad, int64_t ldg, float* dweight,
                                     int64_t lddw, int64_t V, int C, int accumulate, void* stream) {
  MTX_CHECK_ARG(idx && grad && dweight, "embedding_bwd: null pointer");
  MTX_CHECK_SHAPE(n >= 0 && C >= 1 && V >= 1 && V < (1 << 30) && ldg >= C && lddw >= C, "embedding_bwd: bad shape");
  hipLaunchKernelGGL(embed_scatter_kernel, dim3((unsigned)V, (C + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), idx, grad, ldg, dweight, lddw, n, C, accumulate ? 1 : 0);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_onehot_f32(const int64_t* idx, int64_t n, int64_t V, float* out, void* stream) {
  MTX_CHECK_ARG(idx && out, "onehot: null pointer");
  MTX_CHECK_SHAPE(n >= 0 && V >= 1, "onehot: bad shape");
  if (n == 0) return MTX_OK;
  const int blocks = (int)std::min<int64_t>((n * V + 255) / 256, 16384);
  hipLaunchKernelGGL(onehot_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), idx, n, V, out);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_adam_blocks(const int64_t* sizes, int ntensors, int64_t* block0_out, int64_t* total_blocks) {
  MTX_CHECK_ARG(sizes && block0_out && total_blocks && ntensors >= 0, "adam_blocks: bad argument");
  int64_t b = 0;
  for (int i = 0; i < ntensors; ++i) {
    MTX_CHECK_SHAPE(sizes[i] >= 0, "adam_blocks: negative size");
    block0_out[i] = b;
    b += (sizes[i] + kAdamChunk - 1) / kAdamChunk;
  }
  *total_blocks = b;
  return MTX_OK;
}

extern "C" int mtx_adam_f32(const void* table, int ntensors, int64_t total_blocks, double lr, double beta1,
                            double beta2, double eps, double weight_decay, int step, void* stream) {
  MTX_CHECK_ARG(table && ntensors >= 1, "adam: empty table");
  MTX_CHECK_ARG(step >= 1, "adam: step must be >= 1");
  MTX_CHECK_SHAPE(total_blocks >= 0 && total_blocks < (1LL << 31), "adam: bad block count");
  if (total_blocks == 0) return MTX_OK;
  // scalars rounded to float32 exactly as NumPy does for python-float * float32 array
  const AdamCoef k{(float)lr, (float)beta1, (float)beta2, (float)(1.0 - beta1), (float)(1.0 - beta2),
                   (float)(1.0 - std::pow(beta1, (double)step)), (float)(1.0 - std::pow(beta2, (double)step)),
                   (float)eps, (float)weight_decay};
  hipLaunchKernelGGL(adam_kernel, dim3((unsigned)total_blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const AdamEntry*>(table), ntensors, k);
  MTX_LAUNCHED();
  return MTX_OK;
}
