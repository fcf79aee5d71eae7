// Strided-batched fp32 GEMM on gfx950 MFMA (v_mfma_f32_16x16x4_f32).
//
// Replaces the reference's Tensor.__matmul__ (tensor.py:207-223) forward and
// both backward products (dA = dC @ B^T, dB = A^T @ dC, via strides: a
// transpose is a stride swap, never a copy) and the Linear layer's x @ W + b
// (layers.py:31-37, bias fused into the epilogue).
//
//   C[b] = alpha * A[b] @ B[b] + beta * C[b] + bias      (bias indexed by n)
//
// Every operand is (rows, cols) with a row stride, a column stride and a batch
// stride (batch stride 0 broadcasts).  One of A's strides and one of B's must
// be 1 (the loader vectorises along it); the wrapper copies otherwise.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; block tile BM x BN x 16, each
// wave (BM/2) x (BN/2) built from 16x16 MFMA tiles.  The next k-tile is
// prefetched into registers while the current one is multiplied out of LDS.
// Large-K, small-MN products (weight gradients: K = B*T) are split over K:
// each split writes an fp32 partial tile into the caller's workspace and a
// second kernel sums the partials in a fixed order (deterministic), applying
// alpha, beta and bias.
#include "mtx_common.h"

namespace mtx {
namespace {

constexpr int kGT = 256;  // threads per GEMM workgroup
constexpr int BK = 16;

struct GemmArgs {
  const float* a; int64_t sam, sak, sab;
  const float* b; int64_t sbk, sbn, sbb;
  float* c; int64_t scm, scn, scb;
  const float* bias;
  float* ws;          // split-K partials: [split][batch][M][N] contiguous
  int M, N, K, batch;
  int ksplit, kchunk; // K range of split s: [s*kchunk, min(K, (s+1)*kchunk))
  float alpha, beta;
};

template <int BM, int BN, bool AK, bool BN1>
struct Tiles {
  // per-thread register staging of one k-tile
  static constexpr int A_VEC = BM * BK / 4 / kGT;  // float4 per thread
  static constexpr int B_VEC = BN * BK / 4 / kGT;
};

// Load one k-tile of A (BM x BK) into registers.
// AK: A is contiguous along k (sak == 1); else contiguous along m (sam == 1).
template <int BM, bool AK>
__device__ __forceinline__ void load_a(const GemmArgs& g, const float* __restrict__ A, int m0, int k0,
                                       int kend, f32x4 (&r)[BM * BK / 4 / kGT], int tid) {
  constexpr int NV = BM * BK / 4 / kGT;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if constexpr (AK) {
      const int m = m0 + idx / (BK / 4), k = k0 + (idx % (BK / 4)) * 4;
      if (m < g.M) {
        const float* p = A + (int64_t)m * g.sam + k;
        if (k + 3 < kend && ((((uintptr_t)p) & 15u) == 0)) {
          v = *reinterpret_cast<const f32x4*>(p);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (k + j < kend) v[j] = p[j];
        }
      }
    } else {
      const int k = k0 + idx / (BM / 4), m = m0 + (idx % (BM / 4)) * 4;
      if (k < kend) {
        const float* p = A + (int64_t)k * g.sak + m;
        if (m + 3 < g.M && ((((uintptr_t)p) & 15u) == 0)) {
          v = *reinterpret_cast<const f32x4*>(p);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (m + j < g.M) v[j] = p[j];
        }
      }
    }
    r[i] = v;
  }
}

template <int BM, bool AK>
__device__ __forceinline__ void store_a(float* __restrict__ As, const f32x4 (&r)[BM * BK / 4 / kGT], int tid) {
  constexpr int NV = BM * BK / 4 / kGT;
  constexpr int LD = BM + 4;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    if constexpr (AK) {
      const int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) As[(k + j) * LD + m] = r[i][j];
    } else {
      const int k = idx / (BM / 4), m = (idx % (BM / 4)) * 4;
      *reinterpret_cast<f32x4*>(As + k * LD + m) = r[i];
    }
  }
}

// B tile (BK x BN).  BN1: B contiguous along n (sbn == 1); else along k.
template <int BN, bool BN1>
__device__ __forceinline__ void load_b(const GemmArgs& g, const float* __restrict__ Bp, int n0, int k0,
                                       int kend, f32x4 (&r)[BN * BK / 4 / kGT], int tid) {
  constexpr int NV = BN * BK / 4 / kGT;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BN1) {
      const int k = k0 + idx / (BN / 4), n = n0 + (idx % (BN / 4)) * 4;
      if (k < kend) {
        const float* p = Bp + (int64_t)k * g.sbk + n;
        if (n + 3 < g.N && ((((uintptr_t)p) & 15u) == 0)) {
          v = *reinterpret_cast<const f32x4*>(p);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n + j < g.N) v[j] = p[j];
        }
      }
    } else {
      const int n = n0 + idx / (BK / 4), k = k0 + (idx % (BK / 4)) * 4;
      if (n < g.N) {
        const float* p = Bp + (int64_t)n * g.sbn + k;
        if (k + 3 < kend && ((((uintptr_t)p) & 15u) == 0)) {
          v = *reinterpret_cast<const f32x4*>(p);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (k + j < kend) v[j] = p[j];
        }
      }
    }
    r[i] = v;
  }
}

template <int BN, bool BN1>
__device__ __forceinline__ void store_b(float* __restrict__ Bs, const f32x4 (&r)[BN * BK / 4 / kGT], int tid) {
  constexpr int NV = BN * BK / 4 / kGT;
  constexpr int LD = BN + 4;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    if constexpr (BN1) {
      const int k = idx / (BN / 4), n = (idx % (BN / 4)) * 4;
      *reinterpret_cast<f32x4*>(Bs + k * LD + n) = r[i];
    } else {
      const int n = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) Bs[(k + j) * LD + n] = r[i][j];
    }
  }
}

template <int BM, int BN, bool AK, bool BN1>
__global__ __launch_bounds__(kGT) void gemm_f32_kernel(const GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int LDA = BM + 4, LDB = BN + 4;
  __shared__ __attribute__((aligned(16))) float As[BK * LDA];
  __shared__ __attribute__((aligned(16))) float Bs[BK * LDB];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int n16 = lane & 15, grp = lane >> 4;
  const int wm = (wid >> 1) * WM, wn = (wid & 1) * WN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int zb = blockIdx.z;
  const int bidx = zb % g.batch, split = zb / g.batch;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);

  const float* __restrict__ A = g.a + (int64_t)bidx * g.sab;
  const float* __restrict__ Bp = g.b + (int64_t)bidx * g.sbb;

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = zero4();

  f32x4 ra[BM * BK / 4 / kGT], rb[BN * BK / 4 / kGT];
  if (kbeg < kend) {
    load_a<BM, AK>(g, A, m0, kbeg, kend, ra, tid);
    load_b<BN, BN1>(g, Bp, n0, kbeg, kend, rb, tid);
  }
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    __syncthreads();
    store_a<BM, AK>(As, ra, tid);
    store_b<BN, BN1>(Bs, rb, tid);
    __syncthreads();
    if (k0 + BK < kend) {
      load_a<BM, AK>(g, A, m0, k0 + BK, kend, ra, tid);
      load_b<BN, BN1>(g, Bp, n0, k0 + BK, kend, rb, tid);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[(kk + grp) * LDA + wm + 16 * i + n16];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[(kk + grp) * LDB + wn + 16 * j + n16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // epilogue.  acc[i][j][r] = C[wm+16i+4grp+r][wn+16j+n16]
  if (g.ksplit > 1) {
    float* __restrict__ W = g.ws + ((int64_t)split * g.batch + bidx) * (int64_t)g.M * g.N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn + 16 * j + n16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm + 16 * i + 4 * grp + r;
          if (m < g.M && n < g.N) W[(int64_t)m * g.N + n] = acc[i][j][r];
        }
      }
    return;
  }
  float* __restrict__ Cp = g.c + (int64_t)bidx * g.scb;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn + 16 * j + n16;
      if (n >= g.N) continue;
      const float bv = g.bias ? g.bias[n] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + 16 * i + 4 * grp + r;
        if (m < g.M) {
          float* p = Cp + (int64_t)m * g.scm + (int64_t)n * g.scn;
          float v = g.alpha * acc[i][j][r] + bv;
          if (g.beta != 0.f) v += g.beta * *p;
          *p = v;
        }
      }
    }
}

// Sum the split-K partials in split order; apply alpha, beta, bias.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const GemmArgs g) {
  const int64_t MN = (int64_t)g.M * g.N;
  const int64_t total = MN * g.batch;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int bidx = (int)(i / MN);
    const int64_t e = i % MN;
    const int m = (int)(e / g.N), n = (int)(e % g.N);
    float s = 0.f;
    for (int sp = 0; sp < g.ksplit; ++sp) s += g.ws[((int64_t)sp * g.batch + bidx) * MN + e];
    float* p = g.c + (int64_t)bidx * g.scb + (int64_t)m * g.scm + (int64_t)n * g.scn;
    float v = g.alpha * s + (g.bias ? g.bias[n] : 0.f);
    if (g.beta != 0.f) v += g.beta * *p;
    *p = v;
  }
}

struct Plan {
  int bm, bn, ksplit, kchunk;
};

// Pick the tile and the K split for a problem so that the launch has enough
// workgroups to fill 256 CUs, splitting K only when it is long.
Plan plan_gemm(int M, int N, int K, int batch, size_t ws_bytes) {
  Plan p{128, 128, 1, K};
  auto tiles = [&](int bm, int bn) { return (int64_t)cdiv(M, bm) * cdiv(N, bn) * batch; };
  if (tiles(128, 128) < 512) { p.bm = 64; p.bn = 64; }
  const int64_t t = tiles(p.bm, p.bn);
  if (t < 256 && K >= 1024) {
    int want = (int)std::min<int64_t>(16, (512 + t - 1) / t);
    // each split keeps >= 256 of K
    want = std::min(want, std::max(1, K / 256));
    const size_t need = (size_t)want * batch * (size_t)M * N * sizeof(float);
    if (want > 1 && need <= ws_bytes) {
      p.ksplit = want;
      p.kchunk = cdiv(cdiv(K, want), BK) * BK;
      p.ksplit = cdiv(K, p.kchunk);
    }
  } else if (t < 64 && K >= 128) {
    // skinny products (decode steps: M = sequences): too few output tiles to
    // cover the CUs, so split K into chunks of >= 64
    int want = (int)std::min<int64_t>(16, (256 + t - 1) / t);
    want = std::min(want, K / 64);
    const size_t need = (size_t)want * batch * (size_t)M * N * sizeof(float);
    if (want > 1 && need <= ws_bytes) {
      p.ksplit = want;
      p.kchunk = cdiv(cdiv(K, want), BK) * BK;
      p.ksplit = cdiv(K, p.kchunk);
    }
  }
  return p;
}

template <int BM, int BN>
int launch_tile(const GemmArgs& g, bool ak, bool bn1, hipStream_t st) {
  dim3 grid(cdiv(g.N, BN), cdiv(g.M, BM), g.batch * g.ksplit);
  if (ak && bn1) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, true, true>), grid, dim3(kGT), 0, st, g);
  else if (ak) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, true, false>), grid, dim3(kGT), 0, st, g);
  else if (bn1) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, false, true>), grid, dim3(kGT), 0, st, g);
  else hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, false, false>), grid, dim3(kGT), 0, st, g);
  MTX_LAUNCHED();
  return MTX_OK;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" size_t mtx_gemm_workspace_bytes(int M, int N, int K, int batch) {
  if (M < 1 || N < 1 || K < 1 || batch < 1) return 0;
  Plan p = plan_gemm(M, N, K, batch, (size_t)-1);
  return p.ksplit > 1 ? (size_t)p.ksplit * batch * (size_t)M * N * sizeof(float) : 0;
}

extern "C" int mtx_gemm_f32(int M, int N, int K, int batch,
                            float alpha, const float* a, int64_t sa_m, int64_t sa_k, int64_t sa_b,
                            const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b,
                            float beta, float* c, int64_t sc_m, int64_t sc_n, int64_t sc_b,
                            const float* bias, void* workspace, size_t workspace_bytes,
                            void* stream) {
  MTX_CHECK_SHAPE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "negative GEMM size");
  if (M == 0 || N == 0 || batch == 0) return MTX_OK;
  MTX_CHECK_ARG(c != nullptr, "gemm: null C");
  MTX_CHECK_ARG(K == 0 || (a != nullptr && b != nullptr), "gemm: null A or B");
  MTX_CHECK_ARG(sa_k == 1 || sa_m == 1, "gemm: A needs a unit stride along m or k");
  MTX_CHECK_ARG(sb_n == 1 || sb_k == 1, "gemm: B needs a unit stride along k or n");
  MTX_CHECK_ARG(sc_m >= 0 && sc_n >= 0 && sa_b >= 0 && sb_b >= 0 && sc_b >= 0, "gemm: negative stride");
  MTX_CHECK_SHAPE((int64_t)batch * cdiv(M, 64) < 65535 * 64, "gemm: too many tiles");
  GemmArgs g{a, sa_m, sa_k, sa_b, b, sb_k, sb_n, sb_b, c, sc_m, sc_n, sc_b, bias,
             static_cast<float*>(workspace), M, N, K, batch, 1, K, alpha, beta};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 0) {  // C = beta*C + bias
    g.ksplit = 1;
    g.kchunk = 0;
    return launch_tile<64, 64>(g, true, true, st);
  }
  Plan p = plan_gemm(M, N, K, batch, workspace ? workspace_bytes : 0);
  g.ksplit = p.ksplit;
  g.kchunk = p.kchunk;
  const bool ak = sa_k == 1, bn1 = sb_n == 1;
  int rc = (p.bm == 128) ? launch_tile<128, 128>(g, ak, bn1, st) : launch_tile<64, 64>(g, ak, bn1, st);
  if (rc) return rc;
  if (p.ksplit > 1) {
    const int64_t total = (int64_t)M * N * batch;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(blocks), dim3(256), 0, st, g);
    MTX_LAUNCHED();
  }
  return MTX_OK;
}
