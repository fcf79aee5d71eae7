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

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace mtx {
namespace {

constexpr int kGT = 256;  // threads per GEMM workgroup
#ifndef MTX_GEMM_BK
#define MTX_GEMM_BK 16
#endif
constexpr int BK = MTX_GEMM_BK;  // k-tile depth of the tiled kernel
// split-K planning of long-K products: aim at about MTX_SPLIT_TARGET
// workgroups, each with at least MTX_SPLIT_MINK of K (C2 weight gradients,
// K = 16384, summed over the four shapes of a layer: target 256 5.23 ms,
// 512 4.21, 768 3.98, 1024 4.04-4.08 per step)
#ifndef MTX_SPLIT_TARGET
#define MTX_SPLIT_TARGET 768
#endif
#ifndef MTX_SPLIT_MINK
#define MTX_SPLIT_MINK 256
#endif

struct GemmArgs {
  const float* a; int64_t sam, sak, sab;
  const float* b; int64_t sbk, sbn, sbb;
  float* c; int64_t scm, scn, scb;
  const float* bias;
  float* ws;          // split-K partials: [split][batch][M][N] contiguous
  int M, N, K, batch;
  int ksplit, kchunk; // K range of split s: [s*kchunk, min(K, (s+1)*kchunk))
  float alpha, beta;
  // A and B give 16-byte-aligned vectors along their unit-stride dimension
  // at every multiple of 4 (base, other strides and batch strides: set by
  // the host; enables the interior-tile loads)
  int vec_ok;
  // decode-step epilogue (skinny kernel only): act 1 = GELU (tanh form) on
  // the C columns; product columns [nc, N) go to the KV caches instead of C:
  // the first half to kc, the second to vc, at row lengths[m] - 1 of
  // sequence m (row stride cst, sequence stride csb, T rows)
  int act, nc;
  float* kc;
  float* vc;
  int64_t csb, cst;
  int cT;
  const int* lengths;
  // tiled-kernel activation epilogue (mtx_gemm_act_f32): act 1 = GELU, with
  // the pre-activation value also stored to aux when aux != null; act 2 =
  // multiply by GELU'(aux) (aux = the pre-activation read back); act 4 = add
  // aux (a residual stream)
  float* aux;
  int64_t sxm, sxn, sxb;
  // weight-gradient variant (mtx_gemm_wgrad_f32, batch 1): colsum[n] =
  // sum over k of B[k][n] (the bias gradient), added to colsum when
  // colsum_acc; with split K the per-split sums go to the workspace after the
  // C partials, [split][N], and the reduce adds them in split order
  float* colsum;
  int colsum_acc;
  // skinny kernel: write the partial product to ws even when K is not split
  // (the split-K entry points of one range, K <= 16)
  int to_ws;
};

// the value stored at C[m][n] of batch b from the product's value v
__device__ __forceinline__ float epilogue(const GemmArgs& g, float v, int bidx, int m, int n) {
  if (g.act == 1) {
    if (g.aux) g.aux[(int64_t)bidx * g.sxb + (int64_t)m * g.sxm + (int64_t)n * g.sxn] = v;
    return gelu_tanh_fast(v);
  }
  if (g.act == 2) return v * gelu_grad_fast(g.aux[(int64_t)bidx * g.sxb + (int64_t)m * g.sxm + (int64_t)n * g.sxn]);
  if (g.act == 4) return v + g.aux[(int64_t)bidx * g.sxb + (int64_t)m * g.sxm + (int64_t)n * g.sxn];
  return v;
}

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

// LDS tiles are k-major, [BK][BM] (A) and [BK][BN] (B), unpadded; within row
// k the 16-float column blocks are XOR-permuted by tswz(k).  A wave's
// fragment read takes 16 consecutive columns from each of 4 consecutive
// rows, and the transposing scalar stores write 16 columns x 4 rows 4 apart:
// with the permutation both touch 64 distinct banks (a padded row of BM + 4
// floats gave the reads 4-way conflicts).  Needs BM, BN >= 64.
__device__ __forceinline__ int tswz(int k) { return ((k + (k >> 2)) & 3) << 4; }

template <int BM, bool AK>
__device__ __forceinline__ void store_a(float* __restrict__ As, const f32x4 (&r)[BM * BK / 4 / kGT], int tid) {
  constexpr int NV = BM * BK / 4 / kGT;
  static_assert(BM >= 64, "the LDS permutation spans 64 columns");
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    if constexpr (AK) {
      const int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) As[(k + j) * BM + (m ^ tswz(k + j))] = r[i][j];
    } else {
      const int k = idx / (BM / 4), m = (idx % (BM / 4)) * 4;
      *reinterpret_cast<f32x4*>(As + k * BM + (m ^ tswz(k))) = r[i];
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
  static_assert(BN >= 64, "the LDS permutation spans 64 columns");
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = tid + i * kGT;
    if constexpr (BN1) {
      const int k = idx / (BN / 4), n = (idx % (BN / 4)) * 4;
      *reinterpret_cast<f32x4*>(Bs + k * BN + (n ^ tswz(k))) = r[i];
    } else {
      const int n = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) Bs[(k + j) * BN + (n ^ tswz(k + j))] = r[i][j];
    }
  }
}

template <int BM, int BN, bool AK, bool BN1, int ACT>
__global__ __launch_bounds__(kGT) void gemm_f32_kernel(const GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  __shared__ __attribute__((aligned(16))) float As[BK * BM];
  __shared__ __attribute__((aligned(16))) float Bs[BK * BN];

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
  // ACT 3: column sums of B from the values each lane feeds the MFMAs (lane
  // (grp, n16) sees B[k][wn + 16j + n16] for every k = grp mod 4)
  float csum[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) csum[j] = 0.f;
  // only the waves whose sums are stored (below) add them (wave-uniform)
  const bool cs_wave = blockIdx.y == 0 && __builtin_amdgcn_readfirstlane(wm) == 0;

  constexpr int AV = BM * BK / 4 / kGT, BV = BN * BK / 4 / kGT;
  f32x4 ra[AV], rb[BV];
  // Interior tiles (every row and column in range, 16-byte aligned vectors
  // checked on the host) load whole k tiles without per-element checks,
  // from per-thread offsets computed once; other tiles and the last partial
  // k tile take the checked loaders.
  const bool interior = g.vec_ok && m0 + BM <= g.M && n0 + BN <= g.N;
  int64_t aoff[AV], boff[BV];
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int idx = tid + i * kGT;
    aoff[i] = AK ? (int64_t)(m0 + idx / (BK / 4)) * g.sam + (idx % (BK / 4)) * 4
                 : (int64_t)(idx / (BM / 4)) * g.sak + m0 + (idx % (BM / 4)) * 4;
  }
#pragma unroll
  for (int i = 0; i < BV; ++i) {
    const int idx = tid + i * kGT;
    boff[i] = BN1 ? (int64_t)(idx / (BN / 4)) * g.sbk + n0 + (idx % (BN / 4)) * 4
                  : (int64_t)(n0 + idx / (BK / 4)) * g.sbn + (idx % (BK / 4)) * 4;
  }
  const int64_t ak = AK ? 1 : g.sak, bk = BN1 ? g.sbk : 1;  // k stride of the offsets
  auto fetch = [&](int k0) {
    if (interior && k0 + BK <= kend) {
#pragma unroll
      for (int i = 0; i < AV; ++i) ra[i] = *reinterpret_cast<const f32x4*>(A + aoff[i] + (int64_t)k0 * ak);
#pragma unroll
      for (int i = 0; i < BV; ++i) rb[i] = *reinterpret_cast<const f32x4*>(Bp + boff[i] + (int64_t)k0 * bk);
    } else {
      load_a<BM, AK>(g, A, m0, k0, kend, ra, tid);
      load_b<BN, BN1>(g, Bp, n0, k0, kend, rb, tid);
    }
  };
  if (kbeg < kend) fetch(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    __syncthreads();
    store_a<BM, AK>(As, ra, tid);
    store_b<BN, BN1>(Bs, rb, tid);
    __syncthreads();
    if (k0 + BK < kend) fetch(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[(kk + grp) * BM + ((wm + 16 * i + n16) ^ tswz(kk + grp))];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[(kk + grp) * BN + ((wn + 16 * j + n16) ^ tswz(kk + grp))];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
      if constexpr (ACT == 3) {
        if (cs_wave) {
#pragma unroll
          for (int j = 0; j < TN; ++j) csum[j] += bf[j];
        }
      }
    }
  }

  // ACT 3: the first row of tiles (its waves 0 and 1, which together cover
  // the BN columns) adds the four lane groups' sums and stores them
  if constexpr (ACT == 3) {
    if (cs_wave) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float v = csum[j];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        const int n = n0 + wn + 16 * j + n16;
        if (grp == 0 && n < g.N) {
          if (g.ksplit > 1) {
            g.ws[(int64_t)g.ksplit * g.M * g.N + (int64_t)split * g.N + n] = v;
          } else {
            g.colsum[n] = g.colsum_acc ? g.colsum[n] + v : v;
          }
        }
      }
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
  // the activation is a template parameter, so the plain GEMMs keep their
  // register budget; the GELU-backward reads one tile row's pre-activations
  // (16 values) ahead of their use
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float xa[TN][4];
    if constexpr (ACT == 2) {
      const float* __restrict__ X = g.aux + (int64_t)bidx * g.sxb;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = min(n0 + wn + 16 * j + n16, g.N - 1);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = min(m0 + wm + 16 * i + 4 * grp + r, g.M - 1);
          xa[j][r] = X[(int64_t)m * g.sxm + (int64_t)n * g.sxn];
        }
      }
    }
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
          if constexpr (ACT == 1) {
            if (g.aux) g.aux[(int64_t)bidx * g.sxb + (int64_t)m * g.sxm + (int64_t)n * g.sxn] = v;
            v = gelu_tanh_fast(v);
          } else if constexpr (ACT == 2) {
            v *= gelu_grad_fast(xa[j][r]);
          } else if constexpr (ACT == 4) {
            v += g.aux[(int64_t)bidx * g.sxb + (int64_t)m * g.sxm + (int64_t)n * g.sxn];
          }
          *p = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 products on the bf16 matrix cores (the default for tiles of 128 x 128).
//
// Every fp32 operand value x is split into three bf16 pieces while its tile
// is staged into LDS: x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1)
// (each conversion rounds to nearest even; each difference is exact in fp32),
// so x = x0 + x1 + x2 + r with |r| <= 2^-24 |x|: the pieces carry x's 24-bit
// significand.  A product x*y is accumulated as the six piece products of
// weight >= 2^-16 (x2y0, x1y1, x0y2, x1y0, x0y1, x0y0, smallest first); the
// three dropped ones (x1y2, x2y1, x2y2) weigh at most ~2^-23 |xy| together.
// Each piece product is exact in fp32 and the matrix core adds it into the
// fp32 accumulator, so a dot product's error is the fp32 accumulation error
// (as with fp32 multiply-adds) plus at most ~2^-22 sum|x_k y_k|.  Six
// v_mfma_f32_32x32x16_bf16 (6 x 32 cycles) do the work of sixteen
// v_mfma_f32_16x16x4_f32 (16 x 32 cycles): 2.7x the fp32 matrix rate.
// Non-finite inputs give NaN (x - x0 is Inf - Inf).
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, block tile 128 x 128 x 16,
// wave tile 64 x 64 = 2 x 2 MFMA tiles of 32 x 32.  The next k-tile is
// fetched into registers while the current one is multiplied out of LDS.
// An operand contiguous along k is staged as [piece][row][k] (rows of 16
// bf16, the two 16-byte chunks swapped on rows 8..15 mod 16) and read with
// ds_read_b128; an operand contiguous along its rows (m or n) as
// [piece][k][row] (rows of 160 bf16) and read with gfx950's transposing
// ds_read_b64_tr_b16, so staging never transposes in registers.  Both
// layouts are free of LDS bank conflicts (SQ_LDS_BANK_CONFLICT = 0).  MFMA 32x32x16 operands: lane l holds row l%32 and
// k = 8(l/32) + 0..7; accumulator element e of lane l is
// C[8(e/4) + 4(l/32) + e%4][l%32].
// ---------------------------------------------------------------------------
#ifndef MTX_X3_XCD
#define MTX_X3_XCD 1
#endif
namespace x3 {
constexpr int T = 128;             // tile rows and columns
constexpr int BK = 16;             // k-tile depth (one MFMA k step)
constexpr int LDK = BK;            // row stride (bf16) of a k-contiguous plane
constexpr int LDR = T + 32;        // row stride (bf16) of a row-contiguous plane
// k-contiguous rows hold two 16-byte chunks, swapped on rows 8..15 mod 16:
// a fragment read's 16 rows then cover 16 distinct 16-byte bank groups and
// a staging store's 8 rows x 4 quarters 32 distinct 8-byte ones
__device__ __forceinline__ int kswz(int row) { return ((row >> 3) & 1) * 8; }
constexpr int NV = T * BK / 4 / kGT;  // float4 per thread per operand tile
}  // namespace x3

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ uint32_t pk_bf16(float x, float y) {
  bf16x2 v = {(__bf16)x, (__bf16)y};
  return __builtin_bit_cast(uint32_t, v);
}

// x = h + m + l (+ 2^-24 |x|), for four values, each plane as four bf16
__device__ __forceinline__ void split3(f32x4 v, uint2& h, uint2& m, uint2& l) {
  h.x = pk_bf16(v[0], v[1]);
  h.y = pk_bf16(v[2], v[3]);
  float r0 = v[0] - __uint_as_float(h.x << 16), r1 = v[1] - __uint_as_float(h.x & 0xffff0000u);
  float r2 = v[2] - __uint_as_float(h.y << 16), r3 = v[3] - __uint_as_float(h.y & 0xffff0000u);
  m.x = pk_bf16(r0, r1);
  m.y = pk_bf16(r2, r3);
  r0 -= __uint_as_float(m.x << 16);
  r1 -= __uint_as_float(m.x & 0xffff0000u);
  r2 -= __uint_as_float(m.y << 16);
  r3 -= __uint_as_float(m.y & 0xffff0000u);
  l.x = pk_bf16(r0, r1);
  l.y = pk_bf16(r2, r3);
}

// One operand's 128 x 16 tile (rows = m for A, n for B).  KC: contiguous
// along k in global memory (rows strided by srow); else contiguous along the
// rows (k strided by sk).  Thread slot i covers, KC: row idx/4, k 4(idx%4)..+3;
// else: k idx/32, rows 4(idx%32)..+3 (idx = tid + 256 i).
template <bool KC>
struct X3Stage {
  static constexpr int PS = KC ? x3::T * x3::LDK : x3::BK * x3::LDR;  // plane size (bf16)
  const float* __restrict__ base;
  int64_t srow, sk;
  int rows, r0;
  int64_t off[x3::NV];
  f32x4 r[x3::NV];

  __device__ __forceinline__ void init(const float* b, int64_t s_row, int64_t s_k, int nrows, int row0, int tid) {
    base = b;
    srow = s_row;
    sk = s_k;
    rows = nrows;
    r0 = row0;
#pragma unroll
    for (int i = 0; i < x3::NV; ++i) {
      const int idx = tid + i * kGT;
      off[i] = KC ? (int64_t)(r0 + idx / 4) * srow + 4 * (idx % 4) : (int64_t)(idx / 32) * sk + r0 + 4 * (idx % 32);
    }
  }
  // every row of the tile and every k of [k0, k0+16) in range, float4
  // loads aligned (checked by the caller)
  __device__ __forceinline__ void fetch_fast(int k0) {
#pragma unroll
    for (int i = 0; i < x3::NV; ++i)
      r[i] = *reinterpret_cast<const f32x4*>(base + off[i] + (int64_t)k0 * (KC ? 1 : sk));
  }
  // rows past `rows` and k past kend read as zero; unaligned vectors by element
  __device__ __forceinline__ void fetch_checked(int k0, int kend, int tid) {
#pragma unroll
    for (int i = 0; i < x3::NV; ++i) {
      const int idx = tid + i * kGT;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if constexpr (KC) {
        const int row = r0 + idx / 4, k = k0 + 4 * (idx % 4);
        if (row < rows) {
          const float* p = base + (int64_t)row * srow + k;
          if (k + 3 < kend && (((uintptr_t)p) & 15u) == 0) {
            v = *reinterpret_cast<const f32x4*>(p);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (k + j < kend) v[j] = p[j];
          }
        }
      } else {
        const int k = k0 + idx / 32, row = r0 + 4 * (idx % 32);
        if (k < kend) {
          const float* p = base + (int64_t)k * sk + row;
          if (row + 3 < rows && (((uintptr_t)p) & 15u) == 0) {
            v = *reinterpret_cast<const f32x4*>(p);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (row + j < rows) v[j] = p[j];
          }
        }
      }
      r[i] = v;
    }
  }
  __device__ __forceinline__ void put(__bf16* __restrict__ lds, int tid) const {
#pragma unroll
    for (int i = 0; i < x3::NV; ++i) {
      const int idx = tid + i * kGT;
      const int o = KC ? (idx / 4) * x3::LDK + ((4 * (idx % 4)) ^ x3::kswz(idx / 4))
                       : (idx / 32) * x3::LDR + 4 * (idx % 32);
      uint2 h, m, l;
      split3(r[i], h, m, l);
      *reinterpret_cast<uint2*>(lds + o) = h;
      *reinterpret_cast<uint2*>(lds + PS + o) = m;
      *reinterpret_cast<uint2*>(lds + 2 * PS + o) = l;
    }
  }
  // piece p's MFMA operand for tile rows rb .. rb+31: lane l gets row
  // rb + l%32 and k = 8(l/32) + 0..7
  __device__ __forceinline__ bf16x8 frag(const __bf16* __restrict__ lds, int p, int rb, int lane) const {
    if constexpr (KC) {
      const int row = rb + (lane & 31);
      return *reinterpret_cast<const bf16x8*>(lds + p * PS + row * x3::LDK + ((8 * (lane >> 5)) ^ x3::kswz(row)));
    } else {
      // transposing read: in each 16-lane group G, lane j = 4i + q addresses
      // k row 8(G/2) + i (+4 for the second half) at rows rb + 16(G%2) + 4q;
      // lane j then receives row rb + 16(G%2) + j at those four k
      const int G = lane >> 4, j = lane & 15;
      const __bf16* p0 = lds + p * PS + (8 * (G >> 1) + (j >> 2)) * x3::LDR + rb + 16 * (G & 1) + 4 * (j & 3);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + 4 * x3::LDR));
      const uint2 ul = __builtin_bit_cast(uint2, lo), uh = __builtin_bit_cast(uint2, hi);
      return __builtin_bit_cast(bf16x8, make_uint4(ul.x, ul.y, uh.x, uh.y));
    }
  }
  // ACT 3 column sums: this thread's share of the staged B values, by
  // column (KC: the 4 k of slot i belong to column idx/4; else slot i holds
  // columns 4(idx%32)..+3, the same for every slot)
  __device__ __forceinline__ void colsum_add(float (&cs)[4]) const {
#pragma unroll
    for (int i = 0; i < x3::NV; ++i) {
      if constexpr (KC) {
        cs[i] += (r[i][0] + r[i][1]) + (r[i][2] + r[i][3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) cs[j] += r[i][j];
      }
    }
  }
};

template <bool AK, bool BN1, int ACT>
__global__ __launch_bounds__(kGT, 2) void gemm_x3_kernel(const GemmArgs g) {
  using SA = X3Stage<AK>;
  using SB = X3Stage<!BN1>;  // B^T: rows = n, contiguous along k iff !BN1
  // the operand planes, reused by the epilogue for half the C tile (64 x 128 fp32)
  constexpr int kAB = 3 * (SA::PS + SB::PS) * 2, kEp = 64 * x3::T * 4;
  __shared__ __attribute__((aligned(16))) char smem[kAB > kEp ? kAB : kEp];
  __bf16* As = reinterpret_cast<__bf16*>(smem);
  __bf16* Bs = As + 3 * SA::PS;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int wm = (wid >> 1) * 64, wn = (wid & 1) * 64;
#if MTX_X3_XCD
  // Workgroups are dealt round-robin over the 8 XCDs in dispatch order;
  // give each XCD a contiguous run of row-major tiles, so the column tiles
  // that share an A row panel read it through the same L2
  int tx = blockIdx.x, ty = blockIdx.y, tz = blockIdx.z;
  {
    const int nt = gridDim.x * gridDim.y * gridDim.z;
    if ((nt & 7) == 0) {
      const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
      const int t = (lin & 7) * (nt >> 3) + (lin >> 3);
      tx = t % gridDim.x;
      ty = (t / gridDim.x) % gridDim.y;
      tz = t / (gridDim.x * gridDim.y);
    }
  }
  const int m0 = ty * x3::T, n0 = tx * x3::T;
  const int zb = tz;
#else
  const int m0 = blockIdx.y * x3::T, n0 = blockIdx.x * x3::T;
  const int zb = blockIdx.z;
#endif
  const int bidx = zb % g.batch, split = zb / g.batch;
  const int kbeg = split * g.kchunk;
  const int kend = min(g.K, kbeg + g.kchunk);

  SA sa;
  SB sb;
  sa.init(g.a + (int64_t)bidx * g.sab, g.sam, g.sak, g.M, m0, tid);
  sb.init(g.b + (int64_t)bidx * g.sbb, g.sbn, g.sbk, g.N, n0, tid);
  const bool interior = g.vec_ok && m0 + x3::T <= g.M && n0 + x3::T <= g.N;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // ACT 3: the first row of tiles sums the B columns it stages
  const bool cs_block = ACT == 3 && m0 == 0;
  float cs[4] = {0.f, 0.f, 0.f, 0.f};

  // one k-tile: stage the fetched values, request the next tile (pref),
  // multiply out of LDS
  auto tile = [&](auto&& pref) {
    __syncthreads();
    sa.put(As, tid);
    sb.put(Bs, tid);
    if constexpr (ACT == 3) {
      if (cs_block) sb.colsum_add(cs);
    }
    __syncthreads();
    pref();
    bf16x8 a[3][2], b[3][2];
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        a[p][i] = sa.frag(As, p, wm + 32 * i, lane);
        b[p][i] = sb.frag(Bs, p, wn + 32 * i, lane);
      }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x16 c = acc[i][j];
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2][i], b[0][j], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][i], b[1][j], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[2][j], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][i], b[0][j], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[1][j], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][i], b[0][j], c, 0, 0, 0);
        acc[i][j] = c;
      }
  };
  auto checked_next = [&](int kn) {
    if (kn < kend) {
      sa.fetch_checked(kn, kend, tid);
      sb.fetch_checked(kn, kend, tid);
    }
  };
  int k0 = kbeg;
  if (interior) {
    // whole k-tiles through the unchecked loads in a branch-free loop; the
    // last whole tile and a ragged tail after it
    const int kfull = kbeg + (kend - kbeg) / x3::BK * x3::BK;
    if (k0 < kfull) {
      sa.fetch_fast(k0);
      sb.fetch_fast(k0);
    } else {
      checked_next(k0);
    }
    for (; k0 + x3::BK < kfull; k0 += x3::BK)
      tile([&] {
        sa.fetch_fast(k0 + x3::BK);
        sb.fetch_fast(k0 + x3::BK);
      });
  } else {
    checked_next(k0);
  }
  for (; k0 < kend; k0 += x3::BK) tile([&] { checked_next(k0 + x3::BK); });

  if constexpr (ACT == 3) {
    // reduce the per-thread column sums through LDS (As is free after the
    // barrier): KC: 4 threads per column, else 8 threads per 4 columns;
    // contributors are added in a fixed order
    if (cs_block) {
      float* red = reinterpret_cast<float*>(As);  // [8][128]
      __syncthreads();
      if constexpr (!BN1) {
#pragma unroll
        for (int i = 0; i < x3::NV; ++i) {
          const int idx = tid + i * kGT;
          red[(idx % 4) * x3::T + idx / 4] = cs[i];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[(tid / 32) * x3::T + 4 * (tid % 32) + j] = cs[j];
      }
      __syncthreads();
      if (tid < x3::T) {
        constexpr int NC = BN1 ? 8 : 4;
        float v = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) v += red[c * x3::T + tid];
        const int n = n0 + tid;
        if (n < g.N) {
          if (g.ksplit > 1) g.ws[(int64_t)g.ksplit * g.M * g.N + (int64_t)split * g.N + n] = v;
          else g.colsum[n] = g.colsum_acc ? g.colsum[n] + v : v;
        }
      }
    }
  }

  // Epilogue, in two halves of 64 rows: the waves put acc[half] into LDS
  // (row r of the half holds tile row 64(r/32) + 32 half + r%32; columns
  // XOR-permuted by 32 on rows 4..7 mod 8, so the two rows a store
  // instruction writes use disjoint banks), then each thread finishes float4
  // runs of C rows: coalesced loads and stores, no per-element addresses.
  // acc[i][j][e] = tile element (wm + 32i + 8(e/4) + 4(lane/32) + e%4, wn + 32j + lane%32).
  float* ep = reinterpret_cast<float*>(smem);
  const int lr = lane & 31, lh = lane >> 5;
  const bool to_ws = g.ksplit > 1;
  float* W = g.ws + ((int64_t)split * g.batch + bidx) * (int64_t)g.M * g.N;
  float* Cp = g.c + (int64_t)bidx * g.scb;
  float* X = g.aux + (int64_t)bidx * g.sxb;
  const bool rd_c = !to_ws && g.beta != 0.f;
  const bool use_x = !to_ws && (ACT == 2 || ACT == 4 || (ACT == 1 && g.aux != nullptr));
  // whole float4 runs of C (and aux) are aligned vectors
  const bool cvec = to_ws ? (g.N % 4 == 0)
                          : (g.scn == 1 && g.scm % 4 == 0 && g.scb % 4 == 0 && (((uintptr_t)g.c) & 15u) == 0 &&
                             (!use_x || (g.sxn == 1 && g.sxm % 4 == 0 && g.sxb % 4 == 0 &&
                                         (((uintptr_t)g.aux) & 15u) == 0)));
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = (wm >> 1) + 8 * (e >> 2) + 4 * lh + (e & 3);
        ep[r * x3::T + ((wn + 32 * j + lr) ^ ((r & 4) << 3))] = acc[half][j][e];
      }
    __syncthreads();
#pragma unroll 2
    for (int q = 0; q < 8; ++q) {
      const int idx = tid + q * kGT;
      const int r = idx >> 5, c = 4 * (idx & 31);
      const int m = m0 + 64 * (r >> 5) + 32 * half + (r & 31);
      const int n = n0 + c;
      if (m >= g.M || n >= g.N) continue;
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(ep + r * x3::T + (c ^ ((r & 4) << 3)));
      const int nv = min(4, g.N - n);
      if (to_ws) {
        float* w = W + (int64_t)m * g.N + n;
        if (cvec && nv == 4) {
          *reinterpret_cast<f32x4*>(w) = a4;
        } else {
          for (int t = 0; t < nv; ++t) w[t] = a4[t];
        }
        continue;
      }
      float* cp = Cp + (int64_t)m * g.scm + (int64_t)n * g.scn;
      float* xp = X + (int64_t)m * g.sxm + (int64_t)n * g.sxn;
      f32x4 v, old = {0.f, 0.f, 0.f, 0.f}, xa = {0.f, 0.f, 0.f, 0.f}, bv = {0.f, 0.f, 0.f, 0.f};
      const bool vec = cvec && nv == 4;
      if (vec) {
        if (rd_c) old = *reinterpret_cast<const f32x4*>(cp);
        if constexpr (ACT == 2 || ACT == 4) xa = *reinterpret_cast<const f32x4*>(xp);
      } else {
        for (int t = 0; t < nv; ++t) {
          if (rd_c) old[t] = cp[(int64_t)t * g.scn];
          if constexpr (ACT == 2 || ACT == 4) xa[t] = xp[(int64_t)t * g.sxn];
        }
      }
      if (g.bias) {
        for (int t = 0; t < nv; ++t) bv[t] = g.bias[n + t];
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float u = g.alpha * a4[t] + bv[t];
        if (rd_c) u += g.beta * old[t];
        v[t] = u;
      }
      if constexpr (ACT == 1) {
        if (g.aux) {
          if (vec) *reinterpret_cast<f32x4*>(xp) = v;
          else
            for (int t = 0; t < nv; ++t) xp[(int64_t)t * g.sxn] = v[t];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = gelu_tanh_fast(v[t]);
      } else if constexpr (ACT == 2) {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] *= gelu_grad_fast(xa[t]);
      } else if constexpr (ACT == 4) {
        v += xa;
      }
      if (vec) *reinterpret_cast<f32x4*>(cp) = v;
      else
        for (int t = 0; t < nv; ++t) cp[(int64_t)t * g.scn] = v[t];
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny products: M <= 64 rows (a decode step's sequences), K <= 4096 (in
// up to 8 ranges of 512, one workgroup each, when longer than 512).
// One workgroup of 16 waves owns 16 output columns for every row; the waves
// split K into 16-wide slices dealt round-robin, and their partial tiles are
// summed through LDS in wave order (deterministic, one launch, no split-K
// workspace).  Within a slice the lane of group grp supplies, to the four
// MFMA steps s = 0..3, k = 4*grp + s for both A and B (the same k on both
// sides, so each MFMA contracts over four distinct k and the four steps
// cover the slice); A's four values are then one 16-byte load when A is
// contiguous along k.  Each wave loads kSkG slices before multiplying them
// (one when A needs scalar loads).
// ---------------------------------------------------------------------------
#ifndef MTX_SKINNY_WAVES
#define MTX_SKINNY_WAVES 16
#endif
#ifndef MTX_SKINNY_INFLIGHT
#define MTX_SKINNY_INFLIGHT 1
#endif
constexpr int kSkW = MTX_SKINNY_WAVES;     // waves per workgroup
constexpr int kSkT = kSkW * 64;            // threads per workgroup
constexpr int kSkG = MTX_SKINNY_INFLIGHT;  // slices in flight per wave
// every workgroup reads all of its K range of A (M x K) through its CU, so a
// longer K is split over workgroups of at most kSkMaxK each (grid.z), whose
// partial tiles gemm_splitk_reduce sums in split order (measured at M = 64:
// K = 384 one launch 5.9 us against 8.9 us for tiled split-K + reduce;
// K = 1536 unsplit 16 us)
constexpr int kSkMaxM = 64, kSkMaxK = 512, kSkMaxSplit = 8;

// four values at k..k+3 along a dimension of stride sk; V: the host has
// checked that the operand is contiguous along k, 16-byte aligned at every
// k multiple of 4, and K % 4 == 0, so a k group is either whole or past K
template <bool V>
__device__ __forceinline__ f32x4 load4_k(const float* __restrict__ p, int64_t sk, int k, int K, bool ok) {
  f32x4 x = zero4();
  if constexpr (V) {
    if (ok && k < K) x = *reinterpret_cast<const f32x4*>(p);
  } else {
    if (ok) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (k + j < K) x[j] = p[(int64_t)j * sk];
    }
  }
  return x;
}

template <bool AV, bool BV>
__global__ __launch_bounds__(kSkT) void gemm_skinny_kernel(const GemmArgs g) {
  __shared__ float red[kSkW][kSkMaxM * 16];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int n16 = lane & 15, grp = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int bidx = blockIdx.y;
  const int split = blockIdx.z;
  const int n = n0 + n16;
  const bool nok = n < g.N;
  // this workgroup's 16-wide k slices (kchunk is a multiple of 16)
  const int sbeg = split * (g.kchunk / 16);
  const int nsl = min((g.K + 15) / 16, sbeg + g.kchunk / 16);
  // lane bases: row 16i + n16 of A (i = 0..3 by a row offset of 16 rows),
  // column n of B, both at k = 4 * grp
  const float* __restrict__ Ab = g.a + (int64_t)bidx * g.sab + (int64_t)n16 * g.sam + (int64_t)(4 * grp) * g.sak;
  const float* __restrict__ Bb = g.b + (int64_t)bidx * g.sbb + (int64_t)n * g.sbn + (int64_t)(4 * grp) * g.sbk;
  const int64_t a16 = 16 * g.sam;
  // slices in flight: A with four scalar loads per group needs the registers
  constexpr int G = AV ? kSkG : 1;

  f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = zero4();
  for (int s0 = sbeg + wid; s0 < nsl; s0 += G * kSkW) {
    f32x4 af[G][4], bf[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int kb = (s0 + j * kSkW) * 16;  // past K after the last slice: zeros
      if (G > 1 && s0 + j * kSkW >= nsl) {       // past this split's range
        af[j][0] = af[j][1] = af[j][2] = af[j][3] = bf[j] = zero4();
        continue;
      }
      const int k = kb + 4 * grp;
      const float* pa = Ab + (int64_t)kb * g.sak;
#pragma unroll
      for (int i = 0; i < 4; ++i) af[j][i] = load4_k<AV>(pa + i * a16, g.sak, k, g.K, 16 * i + n16 < g.M);
      bf[j] = load4_k<BV>(Bb + (int64_t)kb * g.sbk, g.sbk, k, g.K, nok);
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[j][i][s], bf[j][s], acc[i], 0, 0, 0);
  }
  // acc[i][r] = partial C[16i + 4grp + r][n16]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wid][(16 * i + 4 * grp + r) * 16 + n16] = acc[i][r];
  __syncthreads();
#pragma unroll
  for (int e = tid; e < kSkMaxM * 16; e += kSkT) {
    const int row = e >> 4, col = n0 + (e & 15);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kSkW; ++w) v += red[w][e];
    if (row < g.M && col < g.N && (g.ksplit > 1 || g.to_ws)) {
      g.ws[((int64_t)split * g.batch + bidx) * g.M * g.N + (int64_t)row * g.N + col] = v;
    } else if (row < g.M && col < g.N) {
      float o = g.alpha * v + (g.bias ? g.bias[col] : 0.f);
      if (col < g.nc) {
        float* p = g.c + (int64_t)bidx * g.scb + (int64_t)row * g.scm + (int64_t)col * g.scn;
        if (g.beta != 0.f) o += g.beta * *p;
        if (g.act == 1) o = gelu_tanh(o);
        *p = o;
      } else {
        const int half = (g.N - g.nc) >> 1;
        const int j = col - g.nc;
        float* cache = j < half ? g.kc : g.vc;
        const int jj = j < half ? j : j - half;
        const int t = g.lengths[row] - 1;
        if (t >= 0 && t < g.cT) cache[(int64_t)row * g.csb + (int64_t)t * g.cst + jj] = o;
      }
    }
  }
}

// operand contiguous along k with every 4-aligned k group 16-byte aligned
bool k_vec(const float* p, int64_t s_row, int64_t s_k, int64_t s_batch, int K) {
  return s_k == 1 && K % 4 == 0 && (((uintptr_t)p) & 15u) == 0 && s_row % 4 == 0 && s_batch % 4 == 0;
}

bool use_skinny(int M, int K) { return M <= kSkMaxM && K <= kSkMaxK; }
// K splits of the skinny kernel for an M x K activation, 0 when it does not apply
int skinny_splits(int M, int K) {
  if (M > kSkMaxM || K > kSkMaxK * kSkMaxSplit) return 0;
  return cdiv(K, kSkMaxK);
}

// Column sums of B (batch 1) for the weight-gradient entry point when its
// product takes the skinny kernel (M <= 64): 16 columns x 16 k lanes per
// workgroup, the lanes' sums added in lane order.
__global__ __launch_bounds__(256) void gemm_colsum_kernel(const GemmArgs g) {
  __shared__ float part[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int n = blockIdx.x * 16 + tx;
  float s = 0.f;
  if (n < g.N) {
    const float* __restrict__ col = g.b + (int64_t)n * g.sbn;
#pragma unroll 8
    for (int k = ty; k < g.K; k += 16) s += col[(int64_t)k * g.sbk];
  }
  part[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && n < g.N) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += part[k][tx];
    g.colsum[n] = g.colsum_acc ? g.colsum[n] + t : t;
  }
}

// Sum the split-K partials in split order; apply alpha, beta, bias.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const GemmArgs g) {
  const int64_t MN = (int64_t)g.M * g.N;
  const int64_t total = MN * g.batch;
  // indices past the C elements are the weight-gradient variant's column
  // sums (batch 1), on threads of their own
  const int64_t extra = g.colsum ? g.N : 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total + extra;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (i >= total) {
      const int64_t n = i - total;
      float s = 0.f;
#pragma unroll 8
      for (int sp = 0; sp < g.ksplit; ++sp) s += g.ws[(int64_t)g.ksplit * MN + (int64_t)sp * g.N + n];
      g.colsum[n] = g.colsum_acc ? g.colsum[n] + s : s;
      continue;
    }
    const int bidx = (int)(i / MN);
    const int64_t e = i % MN;
    const int m = (int)(e / g.N), n = (int)(e % g.N);
    float s = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < g.ksplit; ++sp) s += g.ws[((int64_t)sp * g.batch + bidx) * MN + e];
    float* p = g.c + (int64_t)bidx * g.scb + (int64_t)m * g.scm + (int64_t)n * g.scn;
    float v = g.alpha * s + (g.bias ? g.bias[n] : 0.f);
    if (g.beta != 0.f) v += g.beta * *p;
    *p = epilogue(g, v, bidx, m, n);
  }
}

// The split-K reduce of a skinny product followed by LayerNorm of the result
// rows (a decode step's "x += h @ W + b, then ln(x)" in one launch): one
// wave per row.  Per element the arithmetic of gemm_splitk_reduce (partials
// added in split order, then alpha, bias, beta * C), then the row
// statistics of layernorm_fwd_kernel on the values just stored, so C and y
// equal the two-launch sequence's.  Every load of the row is issued before
// the first store (a store in between would order each element's loads
// after it), with the split count KS fixed at compile time.
template <int VPL, int KS>
__global__ __launch_bounds__(64) void splitk_reduce_ln_kernel(const GemmArgs g, const float* __restrict__ gamma,
                                                              const float* __restrict__ beta_ln, float eps,
                                                              float* __restrict__ y, int64_t ldy) {
  const int m = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t MN = (int64_t)g.M * g.N;
  float v[VPL], r[VPL], bb[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int n = lane + 64 * i;
    const bool ok = n < g.N;
    const int64_t e = ok ? (int64_t)m * g.N + n : 0;
    float part[KS];
#pragma unroll
    for (int sp = 0; sp < KS; ++sp) part[sp] = g.ws[(int64_t)sp * MN + e];
    float s = 0.f;
#pragma unroll
    for (int sp = 0; sp < KS; ++sp) s += part[sp];
    v[i] = s;
    r[i] = ok && g.beta != 0.f ? g.c[(int64_t)m * g.scm + (int64_t)n * g.scn] : 0.f;
    bb[i] = ok && g.bias ? g.bias[n] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int n = lane + 64 * i;
    float t = g.alpha * v[i] + bb[i];
    if (g.beta != 0.f) t += g.beta * r[i];
    v[i] = n < g.N ? t : 0.f;
    if (n < g.N) g.c[(int64_t)m * g.scm + (int64_t)n * g.scn] = t;
  }
  float mean, sd;
  ln_stats<VPL>(v, lane, g.N, eps, mean, sd);
  float* yr = y + (int64_t)m * ldy;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int n = lane + 64 * i;
    if (n < g.N) yr[n] = ln_apply(v[i], sd, gamma[n], beta_ln[n]);
  }
}

template <int VPL>
void launch_reduce_ln(const GemmArgs& g, const float* gamma, const float* beta_ln, float eps, float* y,
                      int64_t ldy, hipStream_t st) {
  const dim3 grid(g.M), block(64);
#define RLN(KS) hipLaunchKernelGGL((splitk_reduce_ln_kernel<VPL, KS>), grid, block, 0, st, g, gamma, beta_ln, eps, y, ldy)
  switch (g.ksplit) {
    case 1: RLN(1); break;
    case 2: RLN(2); break;
    case 3: RLN(3); break;
    case 4: RLN(4); break;
    case 5: RLN(5); break;
    case 6: RLN(6); break;
    case 7: RLN(7); break;
    default: RLN(8); break;
  }
#undef RLN
}

struct Plan {
  int bm, bn, ksplit, kchunk;
};

// Pick the tile and the K split for a problem so that the launch has enough
// workgroups to fill 256 CUs, splitting K only when it is long.
Plan plan_gemm(int M, int N, int K, int batch, size_t ws_bytes) {
  Plan p{128, 128, 1, K};
  auto tiles = [&](int bm, int bn) { return (int64_t)cdiv(M, bm) * cdiv(N, bn) * batch; };
  // Long-K products with both sides >= 128 (weight gradients, K = B*T) keep
  // 128x128 tiles and split K further: with 64x64 tiles every tile row and
  // column re-reads its operand panel from beyond L2, twice the traffic.
  const bool longk = K >= 4096 && M >= 128 && N >= 128;
  // 128x128 tiles only when they fill whole rounds of the 256 CUs: a last,
  // partly filled round of these long-running tiles costs more than the
  // smaller tiles' extra operand traffic (16384 x 1152, K = 384: 179 us with
  // 1152 = 4.5 x 256 tiles of 128x128)
  const int64_t t128 = tiles(128, 128);
  if (!longk && (t128 < 512 || t128 % 256 != 0)) { p.bm = 64; p.bn = 64; }
  const int64_t t = tiles(p.bm, p.bn);
  if (t < 256 && K >= 1024) {
    // up to 64 splits for K >= 4096 (partials: want x M x N floats)
    int want = (int)std::min<int64_t>(K >= 4096 ? 64 : 16, (MTX_SPLIT_TARGET + t - 1) / t);
    // each split keeps >= MTX_SPLIT_MINK of K
    want = std::min(want, std::max(1, K / MTX_SPLIT_MINK));
    const size_t need = (size_t)want * batch * (size_t)(M + 1) * N * sizeof(float);
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

template <int BM, int BN, int ACT>
void launch_tile_act(const GemmArgs& g, bool ak, bool bn1, hipStream_t st) {
  dim3 grid(cdiv(g.N, BN), cdiv(g.M, BM), g.batch * g.ksplit);
  if (ak && bn1) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, true, true, ACT>), grid, dim3(kGT), 0, st, g);
  else if (ak) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, true, false, ACT>), grid, dim3(kGT), 0, st, g);
  else if (bn1) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, false, true, ACT>), grid, dim3(kGT), 0, st, g);
  else hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, false, false, ACT>), grid, dim3(kGT), 0, st, g);
}

// the activation epilogue applies only when the tile kernel writes C itself
// (unsplit K); with split K the reduce kernel applies it
template <int BM, int BN>
int launch_tile(const GemmArgs& g, bool ak, bool bn1, hipStream_t st) {
  const int act = g.ksplit > 1 ? 0 : g.act;
  if (g.colsum) launch_tile_act<BM, BN, 3>(g, ak, bn1, st);
  else if (act == 1) launch_tile_act<BM, BN, 1>(g, ak, bn1, st);
  else if (act == 2) launch_tile_act<BM, BN, 2>(g, ak, bn1, st);
  else if (act == 4) launch_tile_act<BM, BN, 4>(g, ak, bn1, st);
  else launch_tile_act<BM, BN, 0>(g, ak, bn1, st);
  MTX_LAUNCHED();
  return MTX_OK;
}

// Which kernel computes fp32 products of at least 128 x 128 (mtx_gemm_set_mode):
// MTX_GEMM_BF16X3 (default) the three-piece bf16 split on the bf16 matrix
// cores, MTX_GEMM_FP32 the fp32 MFMA tile kernel.  Smaller products, and
// the decode step's skinny ones, always take the fp32 kernels.
std::atomic<int> g_gemm_mode{MTX_GEMM_BF16X3};

// Products below 2^27 multiply-adds (the C0 model's 512-row ones: a handful
// of 128 x 128 tiles, latency bound) stay on the fp32 kernel's 64 x 64
// tiles: on the split kernel the C0 training step took 0.445 ms against
// 0.379 ms.
// Nor do products whose 128 x 128 tiles leave part of the 256 CUs idle
// while K is too short to split (< 1024): at M = 2048 (a prefill over 64
// prompts of 32 tokens) the fp32 kernel's 64 x 64 tiles took 28.5, 17.3 and
// 32.0 us for q/k/v (N = 1152), out_proj (N = 384, + residual) and fc1 + GELU
// (N = 1536), all K = 384, against 36.9, 35.7 and 41.6 us on 144, 48 and 192
// split-kernel tiles.
bool use_x3(int M, int N, int K, int batch) {
  if (g_gemm_mode.load(std::memory_order_relaxed) != MTX_GEMM_BF16X3 || M < 128 || N < 128 ||
      (int64_t)M * N * K * batch < ((int64_t)1 << 27))
    return false;
  const int64_t tiles = (int64_t)cdiv(M, x3::T) * cdiv(N, x3::T) * batch;
  return tiles >= 256 || K >= 1024;
}

// Split K only when the 128 x 128 tiles leave the CUs idle (weight gradients,
// K = B*T): aim at MTX_X3_SPLIT_TARGET workgroups (two fit a CU), each split
// keeping >= MTX_SPLIT_MINK of K.
#ifndef MTX_X3_SPLIT_TARGET
#define MTX_X3_SPLIT_TARGET 576
#endif
Plan plan_x3(int M, int N, int K, int batch, size_t ws_bytes) {
  Plan p{x3::T, x3::T, 1, K};
  const int64_t t = (int64_t)cdiv(M, x3::T) * cdiv(N, x3::T) * batch;
  if (t < 256 && K >= 1024) {
    int want = (int)std::min<int64_t>(K >= 4096 ? 64 : 16, (MTX_X3_SPLIT_TARGET + t - 1) / t);
    want = std::min(want, std::max(1, K / MTX_SPLIT_MINK));
    const size_t need = (size_t)want * batch * (size_t)(M + 1) * N * sizeof(float);
    if (want > 1 && need <= ws_bytes) {
      p.kchunk = cdiv(cdiv(K, want), x3::BK) * x3::BK;
      p.ksplit = cdiv(K, p.kchunk);
    }
  }
  return p;
}

template <int ACT>
void launch_x3_act(const GemmArgs& g, bool ak, bool bn1, hipStream_t st) {
  const dim3 grid(cdiv(g.N, x3::T), cdiv(g.M, x3::T), g.batch * g.ksplit);
  if (ak && bn1) hipLaunchKernelGGL((gemm_x3_kernel<true, true, ACT>), grid, dim3(kGT), 0, st, g);
  else if (ak) hipLaunchKernelGGL((gemm_x3_kernel<true, false, ACT>), grid, dim3(kGT), 0, st, g);
  else if (bn1) hipLaunchKernelGGL((gemm_x3_kernel<false, true, ACT>), grid, dim3(kGT), 0, st, g);
  else hipLaunchKernelGGL((gemm_x3_kernel<false, false, ACT>), grid, dim3(kGT), 0, st, g);
}

// as launch_tile: with split K the reduce kernel applies the activation
int launch_x3(const GemmArgs& g, bool ak, bool bn1, hipStream_t st) {
  const int act = g.ksplit > 1 ? 0 : g.act;
  if (g.colsum) launch_x3_act<3>(g, ak, bn1, st);
  else if (act == 1) launch_x3_act<1>(g, ak, bn1, st);
  else if (act == 2) launch_x3_act<2>(g, ak, bn1, st);
  else if (act == 4) launch_x3_act<4>(g, ak, bn1, st);
  else launch_x3_act<0>(g, ak, bn1, st);
  MTX_LAUNCHED();
  return MTX_OK;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" size_t mtx_gemm_workspace_bytes(int M, int N, int K, int batch) {
  if (M < 1 || N < 1 || K < 1 || batch < 1) return 0;
  // The skinny kernel serves plain products with M <= 64; the same shape with
  // an activation epilogue (mtx_gemm_act_f32) or column sums goes to the tile
  // kernel, so the size covers both plans.
  const int sp = skinny_splits(M, K);
  const size_t skinny = sp > 1 ? (size_t)sp * batch * (size_t)M * N * sizeof(float) : 0;
  Plan p = plan_gemm(M, N, K, batch, (size_t)-1);
  // split partials [split][batch][M][N], then the weight-gradient variant's
  // column sums [split][N]
  const size_t tiled = p.ksplit > 1 ? (size_t)p.ksplit * batch * (size_t)(M + 1) * N * sizeof(float) : 0;
  // the bf16-split kernel's plan (either mode may be set when the product runs)
  Plan q = plan_x3(M, N, K, batch, (size_t)-1);
  const size_t split3 = q.ksplit > 1 ? (size_t)q.ksplit * batch * (size_t)(M + 1) * N * sizeof(float) : 0;
  return std::max({skinny, tiled, split3});
}

extern "C" int mtx_gemm_set_mode(int mode) {
  MTX_CHECK_ARG(mode == MTX_GEMM_FP32 || mode == MTX_GEMM_BF16X3,
                "gemm mode %d must be MTX_GEMM_FP32 (0) or MTX_GEMM_BF16X3 (1)", mode);
  g_gemm_mode.store(mode);
  return MTX_OK;
}

extern "C" int mtx_gemm_get_mode(void) { return g_gemm_mode.load(); }

namespace {
int gemm_impl(int M, int N, int K, int batch, float alpha, const float* a, int64_t sa_m, int64_t sa_k,
              int64_t sa_b, const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b, float beta, float* c,
              int64_t sc_m, int64_t sc_n, int64_t sc_b, const float* bias, int act, float* aux, int64_t sx_m,
              int64_t sx_n, int64_t sx_b, void* workspace, size_t workspace_bytes, void* stream,
              float* colsum = nullptr, int colsum_acc = 0) {
  MTX_CHECK_SHAPE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "negative GEMM size");
  if (M == 0 || N == 0 || batch == 0) return MTX_OK;
  MTX_CHECK_ARG(c != nullptr, "gemm: null C");
  MTX_CHECK_ARG(K == 0 || (a != nullptr && b != nullptr), "gemm: null A or B");
  // (an empty K leaves A and B unread, whatever their strides)
  MTX_CHECK_ARG(K == 0 || sa_k == 1 || sa_m == 1, "gemm: A needs a unit stride along m or k");
  MTX_CHECK_ARG(K == 0 || sb_n == 1 || sb_k == 1, "gemm: B needs a unit stride along k or n");
  MTX_CHECK_ARG(sc_m >= 0 && sc_n >= 0 && sa_b >= 0 && sb_b >= 0 && sc_b >= 0, "gemm: negative stride");
  MTX_CHECK_SHAPE((int64_t)batch * cdiv(M, 64) < 65535 * 64, "gemm: too many tiles");
  GemmArgs g{a, sa_m, sa_k, sa_b, b, sb_k, sb_n, sb_b, c, sc_m, sc_n, sc_b, bias,
             static_cast<float*>(workspace), M, N, K, batch, 1, K, alpha, beta};
  g.nc = N;
  g.aux = aux;
  g.sxm = sx_m;
  g.sxn = sx_n;
  g.sxb = sx_b;
  g.colsum = colsum;
  g.colsum_acc = colsum_acc;
  {
    const bool a_ok = (((uintptr_t)a) & 15u) == 0 && (sa_k == 1 ? sa_m % 4 == 0 : sa_k % 4 == 0) && sa_b % 4 == 0;
    const bool b_ok = (((uintptr_t)b) & 15u) == 0 && (sb_n == 1 ? sb_k % 4 == 0 : sb_n % 4 == 0) && sb_b % 4 == 0;
    g.vec_ok = a_ok && b_ok;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the activation epilogue runs in the tiled kernel and the split-K reduce
  // (the skinny kernel's act field is the decode step's own)
  g.act = act;
  if (K == 0) {  // C = act(beta*C + bias)
    g.ksplit = 1;
    g.kchunk = 0;
    return launch_tile<64, 64>(g, true, true, st);
  }
  if (int sp = act ? 0 : skinny_splits(M, K)) {
    MTX_CHECK_SHAPE(batch < 65536, "gemm: batch too large");
    if (colsum) {  // the skinny kernel and its reduce leave the sums to their own kernel
      hipLaunchKernelGGL(gemm_colsum_kernel, dim3(cdiv(N, 16)), dim3(256), 0, st, g);
      MTX_LAUNCHED();
      g.colsum = nullptr;
    }
    // without room for the partials, one workgroup covers all of K
    if (sp > 1 && (!workspace || workspace_bytes < (size_t)sp * batch * (size_t)M * N * sizeof(float))) sp = 1;
    g.ksplit = sp;
    g.kchunk = sp > 1 ? kSkMaxK : cdiv(K, 16) * 16;
    const bool av = k_vec(a, sa_m, sa_k, sa_b, K), bv = k_vec(b, sb_n, sb_k, sb_b, K);
    const dim3 grid(cdiv(N, 16), batch, sp);
    if (av && bv) hipLaunchKernelGGL((gemm_skinny_kernel<true, true>), grid, dim3(kSkT), 0, st, g);
    else if (av) hipLaunchKernelGGL((gemm_skinny_kernel<true, false>), grid, dim3(kSkT), 0, st, g);
    else if (bv) hipLaunchKernelGGL((gemm_skinny_kernel<false, true>), grid, dim3(kSkT), 0, st, g);
    else hipLaunchKernelGGL((gemm_skinny_kernel<false, false>), grid, dim3(kSkT), 0, st, g);
    MTX_LAUNCHED();
    if (sp > 1) {
      const int64_t total = (int64_t)M * N * batch;
      const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
      hipLaunchKernelGGL(gemm_splitk_reduce, dim3(blocks), dim3(256), 0, st, g);
      MTX_LAUNCHED();
    }
    return MTX_OK;
  }
  const bool ak = sa_k == 1, bn1 = sb_n == 1;
  const bool split3 = use_x3(M, N, K, batch);
  Plan p = split3 ? plan_x3(M, N, K, batch, workspace ? workspace_bytes : 0)
                  : plan_gemm(M, N, K, batch, workspace ? workspace_bytes : 0);
  g.ksplit = p.ksplit;
  g.kchunk = p.kchunk;
  int rc = split3 ? launch_x3(g, ak, bn1, st)
                  : (p.bm == 128) ? launch_tile<128, 128>(g, ak, bn1, st) : launch_tile<64, 64>(g, ak, bn1, st);
  if (rc) return rc;
  if (p.ksplit > 1) {
    const int64_t total = (int64_t)M * N * batch + (colsum ? N : 0);
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(blocks), dim3(256), 0, st, g);
    MTX_LAUNCHED();
  }
  return MTX_OK;
}
}  // namespace

extern "C" int mtx_gemm_f32(int M, int N, int K, int batch,
                            float alpha, const float* a, int64_t sa_m, int64_t sa_k, int64_t sa_b,
                            const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b,
                            float beta, float* c, int64_t sc_m, int64_t sc_n, int64_t sc_b,
                            const float* bias, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return gemm_impl(M, N, K, batch, alpha, a, sa_m, sa_k, sa_b, b, sb_k, sb_n, sb_b, beta, c, sc_m, sc_n, sc_b,
                   bias, 0, nullptr, 0, 0, 0, workspace, workspace_bytes, stream);
}

// workgroups a mtx_gemm_ln_f32 product aims at (by splitting K)
constexpr int kLnWgs = 144;

// The split-K product of mtx_gemm_ln_f32 / mtx_gemm_partials_f32: K cut into
// 2..8 ranges of whole 16-wide slices, as many as bring the launch to about
// kLnWgs workgroups (a projection to N = 384 has only 24 column tiles;
// measured at C4: 96 workgroups 0.327, 144 0.315, 192 0.313-0.317 ms per
// token step against 0.340 with mtx_gemm_f32's ranges); range s's partial
// product A[:, range] @ B[range, :] goes to g.ws + s*M*N.  Sets g.ksplit and
// g.kchunk.
void launch_ln_partials(GemmArgs& g, hipStream_t st) {
  const int want = std::min(kSkMaxSplit, std::max({2, skinny_splits(g.M, g.K), cdiv(kLnWgs, cdiv(g.N, 16))}));
  g.kchunk = cdiv(cdiv(g.K, want), 16) * 16;
  g.ksplit = cdiv(g.K, g.kchunk);
  g.nc = g.N;
  g.to_ws = 1;
  const bool av = k_vec(g.a, g.sam, g.sak, 0, g.K), bv = k_vec(g.b, g.sbn, g.sbk, 0, g.K);
  const dim3 grid(cdiv(g.N, 16), 1, g.ksplit);
  if (av && bv) hipLaunchKernelGGL((gemm_skinny_kernel<true, true>), grid, dim3(kSkT), 0, st, g);
  else if (av) hipLaunchKernelGGL((gemm_skinny_kernel<true, false>), grid, dim3(kSkT), 0, st, g);
  else if (bv) hipLaunchKernelGGL((gemm_skinny_kernel<false, true>), grid, dim3(kSkT), 0, st, g);
  else hipLaunchKernelGGL((gemm_skinny_kernel<false, false>), grid, dim3(kSkT), 0, st, g);
}

extern "C" size_t mtx_gemm_ln_workspace_bytes(int M, int N, int K) {
  if (M < 1 || N < 1 || K < 1 || skinny_splits(M, K) == 0) return 0;
  return (size_t)kSkMaxSplit * M * N * sizeof(float);
}

extern "C" int mtx_gemm_ln_f32(int M, int N, int K, float alpha, const float* a, int64_t sa_m, int64_t sa_k,
                               const float* b, int64_t sb_k, int64_t sb_n, float beta, float* c, int64_t sc_m,
                               const float* bias, const float* ln_gamma, const float* ln_beta, float eps, float* y,
                               int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  MTX_CHECK_SHAPE(M >= 1 && N >= 1 && K >= 1, "gemm_ln: sizes must be >= 1");
  MTX_CHECK_SHAPE(M <= kSkMaxM && K <= kSkMaxK * kSkMaxSplit && N <= 64 * 32,
                  "gemm_ln: needs M <= %d, K <= %d and N <= 2048 (got M=%d, N=%d, K=%d)", kSkMaxM,
                  kSkMaxK * kSkMaxSplit, M, N, K);
  MTX_CHECK_ARG(a && b && c && ln_gamma && ln_beta && y, "gemm_ln: null pointer");
  MTX_CHECK_ARG(sa_k == 1 || sa_m == 1, "gemm_ln: A needs a unit stride along m or k");
  MTX_CHECK_ARG(sb_n == 1 || sb_k == 1, "gemm_ln: B needs a unit stride along k or n");
  MTX_CHECK_ARG(sc_m >= N && ldy >= N, "gemm_ln: C and y rows must hold N values");
  MTX_CHECK_ARG((y >= c + (int64_t)(M - 1) * sc_m + N) || (c >= y + (int64_t)(M - 1) * ldy + N),
                "gemm_ln: y must not overlap C");
  const size_t need = mtx_gemm_ln_workspace_bytes(M, N, K);
  MTX_CHECK_ARG(workspace && workspace_bytes >= need, "gemm_ln: workspace too small (%zu < %zu)", workspace_bytes,
                need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemmArgs g{a, sa_m, sa_k, 0, b, sb_k, sb_n, 0, c, sc_m, 1, 0, bias,
             static_cast<float*>(workspace), M, N, K, 1, 0, 0, alpha, beta};
  launch_ln_partials(g, st);
  MTX_LAUNCHED();
  const int vpl = cdiv(N, 64);
  if (vpl <= 1) launch_reduce_ln<1>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 2) launch_reduce_ln<2>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 4) launch_reduce_ln<4>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 6) launch_reduce_ln<6>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 8) launch_reduce_ln<8>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 12) launch_reduce_ln<12>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else if (vpl <= 16) launch_reduce_ln<16>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  else launch_reduce_ln<32>(g, ln_gamma, ln_beta, eps, y, ldy, st);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_gemm_partials_f32(int M, int N, int K, const float* a, int64_t sa_m, int64_t sa_k,
                                     const float* b, int64_t sb_k, int64_t sb_n, void* workspace,
                                     size_t workspace_bytes, int* nsplit, void* stream) {
  MTX_CHECK_SHAPE(M >= 1 && N >= 1 && K >= 1, "gemm_partials: sizes must be >= 1");
  MTX_CHECK_SHAPE(M <= kSkMaxM && K <= kSkMaxK * kSkMaxSplit && N <= 64 * 32,
                  "gemm_partials: needs M <= %d, K <= %d and N <= 2048 (got M=%d, N=%d, K=%d)", kSkMaxM,
                  kSkMaxK * kSkMaxSplit, M, N, K);
  MTX_CHECK_ARG(a && b && nsplit, "gemm_partials: null pointer");
  MTX_CHECK_ARG(sa_k == 1 || sa_m == 1, "gemm_partials: A needs a unit stride along m or k");
  MTX_CHECK_ARG(sb_n == 1 || sb_k == 1, "gemm_partials: B needs a unit stride along k or n");
  const size_t need = mtx_gemm_ln_workspace_bytes(M, N, K);
  MTX_CHECK_ARG(workspace && workspace_bytes >= need, "gemm_partials: workspace too small (%zu < %zu)",
                workspace_bytes, need);
  GemmArgs g{a, sa_m, sa_k, 0, b, sb_k, sb_n, 0, nullptr, N, 1, 0, nullptr,
             static_cast<float*>(workspace), M, N, K, 1, 0, 0, 1.f, 0.f};
  launch_ln_partials(g, static_cast<hipStream_t>(stream));
  MTX_LAUNCHED();
  *nsplit = g.ksplit;
  return MTX_OK;
}

extern "C" int mtx_gemm_act_f32(int M, int N, int K, int batch,
                                float alpha, const float* a, int64_t sa_m, int64_t sa_k, int64_t sa_b,
                                const float* b, int64_t sb_k, int64_t sb_n, int64_t sb_b,
                                float beta, float* c, int64_t sc_m, int64_t sc_n, int64_t sc_b,
                                const float* bias, int act, float* aux, int64_t sx_m, int64_t sx_n,
                                int64_t sx_b, void* workspace, size_t workspace_bytes, void* stream) {
  MTX_CHECK_ARG(act == 0 || act == 1 || act == 2 || act == 4,
                "gemm_act: act=%d must be 0 (none), 1 (GELU), 2 (GELU backward) or 4 (add aux)", act);
  MTX_CHECK_ARG(act != 2 || aux != nullptr, "gemm_act: act 2 needs the pre-activation aux");
  MTX_CHECK_ARG(act != 4 || (aux != nullptr && aux != c), "gemm_act: act 4 needs a residual aux other than C");
  MTX_CHECK_ARG(sx_m >= 0 && sx_n >= 0 && sx_b >= 0, "gemm_act: negative aux stride");
  return gemm_impl(M, N, K, batch, alpha, a, sa_m, sa_k, sa_b, b, sb_k, sb_n, sb_b, beta, c, sc_m, sc_n, sc_b,
                   bias, act, act ? aux : nullptr, sx_m, sx_n, sx_b, workspace, workspace_bytes, stream);
}

extern "C" int mtx_gemm_wgrad_f32(int M, int N, int K, const float* a, int64_t sa_m, int64_t sa_k,
                                  const float* b, int64_t sb_k, int64_t sb_n, float beta, float* c, int64_t sc_m,
                                  int64_t sc_n, float* dbias, int dbias_accumulate, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  MTX_CHECK_ARG(dbias != nullptr, "gemm_wgrad: null dbias (use mtx_gemm_f32 without a bias gradient)");
  MTX_CHECK_SHAPE(M >= 1 && N >= 1 && K >= 0, "gemm_wgrad: sizes must be M, N >= 1, K >= 0");
  return gemm_impl(M, N, K, 1, 1.f, a, sa_m, sa_k, 0, b, sb_k, sb_n, 0, beta, c, sc_m, sc_n, 0, nullptr, 0,
                   nullptr, 0, 0, 0, workspace, workspace_bytes, stream, dbias, dbias_accumulate ? 1 : 0);
}

extern "C" int mtx_gemm_step_f32(int M, int N, int K, const float* a, int64_t lda, const float* b, int64_t ldb,
                                 float beta, float* c, int64_t ldc, const float* bias, int act, int ncols_c,
                                 float* kcache, float* vcache, int64_t cache_stride_b, int64_t cache_stride_t,
                                 int T, const int* lengths, void* stream) {
  MTX_CHECK_SHAPE(M >= 1 && N >= 1 && K >= 1, "gemm_step: sizes must be >= 1");
  MTX_CHECK_SHAPE(use_skinny(M, K), "gemm_step: needs M <= %d and K <= %d (got M=%d, K=%d)", kSkMaxM, kSkMaxK,
                  M, K);
  MTX_CHECK_ARG(a && b && (ncols_c == 0 || c), "gemm_step: null operand");
  MTX_CHECK_ARG(act == 0 || act == 1, "gemm_step: act must be 0 (none) or 1 (gelu)");
  MTX_CHECK_ARG(ncols_c >= 0 && ncols_c <= N, "gemm_step: ncols_c %d not in [0, N=%d]", ncols_c, N);
  MTX_CHECK_ARG(lda >= K && ldb >= N && (ncols_c == 0 || ldc >= ncols_c), "gemm_step: row strides too small");
  if (ncols_c < N) {
    MTX_CHECK_ARG((N - ncols_c) % 2 == 0, "gemm_step: the cache columns must split evenly into k and v");
    MTX_CHECK_ARG(kcache && vcache && lengths, "gemm_step: null cache or lengths");
    MTX_CHECK_ARG(T >= 1 && cache_stride_t >= (N - ncols_c) / 2 && cache_stride_b >= (int64_t)T * cache_stride_t,
                  "gemm_step: cache strides do not hold (B, T, C) rows");
  }
  GemmArgs g{a, lda, 1, 0, b, ldb, 1, 0, c, ldc, 1, 0, bias, nullptr, M, N, K, 1, 1, cdiv(K, 16) * 16, 1.f, beta};
  g.act = act;
  g.nc = ncols_c;
  g.kc = kcache;
  g.vc = vcache;
  g.csb = cache_stride_b;
  g.cst = cache_stride_t;
  g.cT = T;
  g.lengths = lengths;
  const bool av = k_vec(a, lda, 1, 0, K);
  const dim3 grid(cdiv(N, 16), 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (av) hipLaunchKernelGGL((gemm_skinny_kernel<true, false>), grid, dim3(kSkT), 0, st, g);
  else hipLaunchKernelGGL((gemm_skinny_kernel<false, false>), grid, dim3(kSkT), 0, st, g);
  MTX_LAUNCHED();
  return MTX_OK;
}
