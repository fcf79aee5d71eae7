// Row-wise fused kernels (fp32): softmax, log_softmax, LayerNorm, GELU and
// softmax cross-entropy, forward and backward.
//
// Replaces, per row of the last axis:
//   F.softmax        functional.py:62-78  (optionally with the causal mask of
//                    transformer.py:39-40 applied as exact zeros)
//   F.log_softmax    functional.py:81-97
//   LayerNorm        layers.py:73-89 (biased variance, eps inside the sqrt,
//                    x_hat = diff / std: the 9-node composite in one pass)
//   F.gelu           functional.py:54-59 (tanh approximation with the float32
//                    constants the reference's Tensor(scalar) produces)
//   cross_entropy    loss.py:17-27 (log_softmax + one-hot NLL, mean over N)
// One wave64 per row; rows are independent, so every result is deterministic.
#include "mtx_common.h"

namespace mtx {
namespace {

// visible(j) for causal rows: row r of a stack of (Tq, L) matrices
__device__ __forceinline__ int causal_limit(int64_t row, int causal_tq, int L) {
  if (causal_tq <= 0) return L;
  const int i = (int)(row % causal_tq);
  return min(L, i + (L - causal_tq) + 1);
}

__global__ __launch_bounds__(256) void softmax_fwd_kernel(const float* __restrict__ x, int64_t ldx,
                                                          float* __restrict__ y, int64_t ldy,
                                                          int64_t rows, int L, int causal_tq, int log_mode) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * ldx;
  float* yr = y + row * ldy;
  const int lim = causal_limit(row, causal_tq, L);
  float mx = -INFINITY;
  for (int j = lane; j < lim; j += 64) mx = fmaxf(mx, xr[j]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int j = lane; j < lim; j += 64) s += expf(xr[j] - mx);
  s = wave_sum(s);
  if (log_mode) {
    const float lse = logf(s);
    for (int j = lane; j < L; j += 64) yr[j] = j < lim ? (xr[j] - mx) - lse : -INFINITY;
  } else {
    for (int j = lane; j < L; j += 64) yr[j] = j < lim ? expf(xr[j] - mx) / s : 0.f;
  }
}

// softmax:     dx = y * (dy - sum(y * dy))
// log_softmax: dx = dy - exp(y) * sum(dy)
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const float* __restrict__ y, int64_t ldy,
                                                          const float* __restrict__ dy, int64_t lddy,
                                                          float* __restrict__ dx, int64_t lddx,
                                                          int64_t rows, int L, int log_mode, int accumulate) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* yr = y + row * ldy;
  const float* gr = dy + row * lddy;
  float* dr = dx + row * lddx;
  float s = 0.f;
  if (log_mode) {
    for (int j = lane; j < L; j += 64) s += gr[j];
  } else {
    for (int j = lane; j < L; j += 64) s += yr[j] * gr[j];
  }
  s = wave_sum(s);
  for (int j = lane; j < L; j += 64) {
    float v = log_mode ? gr[j] - expf(yr[j]) * s : yr[j] * (gr[j] - s);
    if (accumulate) v += dr[j];
    dr[j] = v;
  }
}


// LayerNorm forward: y = (x - mean) / sqrt(var + eps) * gamma + beta.
// Saves mean and std per row for the backward.
template <int VPL>  // values per lane held in registers (C <= 64 * VPL)
__global__ __launch_bounds__(256) void layernorm_fwd_kernel(const float* __restrict__ x, int64_t ldx,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            float* __restrict__ y, int64_t ldy,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ std_out,
                                                            int64_t rows, int C, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * ldx;
  float v[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    v[i] = j < C ? xr[j] : 0.f;
  }
  float mean, sd;
  ln_stats<VPL>(v, lane, C, eps, mean, sd);
  float* yr = y + row * ldy;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    if (j < C) yr[j] = ln_apply(v[i], sd, gamma[j], beta[j]);
  }
  if (lane == 0) {
    mean_out[row] = mean;
    std_out[row] = sd;
  }
}

// dx = (1/std) * (g - mean(g) - xh * mean(g * xh)), g = dy * gamma, plus
// add (when set; add may be dx itself: each element is read before the same
// thread writes it, so neither pointer is restrict)
template <int VPL>
__global__ __launch_bounds__(256) void layernorm_bwd_kernel(const float* __restrict__ x, int64_t ldx,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ mean_in,
                                                            const float* __restrict__ std_in,
                                                            const float* __restrict__ dy, int64_t lddy,
                                                            float* dx, int64_t lddx, const float* add,
                                                            int64_t ldadd, int64_t rows, int C) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float mean = mean_in[row], sd = std_in[row];
  const float* xr = x + row * ldx;
  const float* gr = dy + row * lddy;
  float xh[VPL], gg[VPL];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    if (j < C) {
      xh[i] = (xr[j] - mean) / sd;
      gg[i] = gr[j] * gamma[j];
    } else {
      xh[i] = 0.f;
      gg[i] = 0.f;
    }
    s1 += gg[i];
    s2 += gg[i] * xh[i];
  }
  s1 = wave_sum(s1) / (float)C;
  s2 = wave_sum(s2) / (float)C;
  float* dr = dx + row * lddx;
  const float* ar = add ? add + row * ldadd : nullptr;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    if (j < C) {
      float v = (gg[i] - s1 - xh[i] * s2) / sd;
      if (ar) v += ar[j];
      dr[j] = v;
    }
  }
}

// LayerNorm backward with the parameter gradients in the same pass over x and
// dy: block b (8 waves) owns rows [b*chunk, (b+1)*chunk); wave w takes rows
// w, w+8, ... of them, writes dx (if asked) as layernorm_bwd_kernel does, and
// keeps per-column sums of dy * xh (dgamma) and dy (dbeta) in registers.  The
// next row's x, dy (and dx when accumulating) are loaded while the current
// row is reduced.  The eight waves' sums are added pairwise through LDS in a
// fixed order and the block's partials [b][2][C] go to the workspace;
// layernorm_param_combine adds them in block order (deterministic).
// Dynamic LDS: 4 * 2 * C floats.
constexpr int LNP_WAVES = 8;
template <int VPL>
__global__ __launch_bounds__(64 * LNP_WAVES) void layernorm_bwd_param_kernel(
    const float* __restrict__ x, int64_t ldx, const float* __restrict__ gamma, const float* __restrict__ mean_in,
    const float* __restrict__ std_in, const float* __restrict__ dy, int64_t lddy, float* dx, int64_t lddx,
    const float* add, int64_t ldadd, float* __restrict__ ws, int64_t rows, int C, int64_t chunk) {
  extern __shared__ float red[];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r0 = (int64_t)blockIdx.x * chunk, r1 = min(rows, r0 + chunk);
  const bool rd_dx = dx != nullptr && add != nullptr;
  // rows of up to 768 columns keep gamma in registers and prefetch the next
  // row (x, dy and the dx being added to); wider rows would spill
  constexpr bool PF = VPL <= 12;
  float gm[VPL], ag[VPL], ab[VPL], cx[VPL], cg[VPL], cd[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = lane + 64 * i;
    gm[i] = PF && j < C ? gamma[j] : 0.f;
    ag[i] = 0.f;
    ab[i] = 0.f;
  }
  auto load_row = [&](int64_t rr, float (&px)[VPL], float (&pg)[VPL], float (&pd)[VPL]) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      const bool ok = rr < r1 && j < C;
      px[i] = ok ? x[rr * ldx + j] : 0.f;
      pg[i] = ok ? dy[rr * lddy + j] : 0.f;
      pd[i] = PF && ok && rd_dx ? add[rr * ldadd + j] : 0.f;
    }
  };
  int64_t r = r0 + w;
  if constexpr (PF) load_row(r, cx, cg, cd);
  for (; r < r1; r += LNP_WAVES) {
    const float mean = mean_in[r], sd = std_in[r];
    const int64_t rn = r + LNP_WAVES;
    float nx[PF ? VPL : 1], ng[PF ? VPL : 1], nd[PF ? VPL : 1];
    if constexpr (PF) load_row(rn, nx, ng, nd);
    else load_row(r, cx, cg, cd);
    // in place: cx becomes xh = (x - mean) / sd, cg becomes g = dy * gamma
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      const float xh = j < C ? (cx[i] - mean) / sd : 0.f;
      const float g = cg[i] * (PF ? gm[i] : (j < C ? gamma[j] : 0.f));
      s1 += g;
      s2 += g * xh;
      ag[i] += cg[i] * xh;
      ab[i] += cg[i];
      cx[i] = xh;
      cg[i] = g;
    }
    if (dx) {
      s1 = wave_sum(s1) / (float)C;
      s2 = wave_sum(s2) / (float)C;
      float* dr = dx + r * lddx;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int j = lane + 64 * i;
        if (j < C) {
          float v = (cg[i] - s1 - cx[i] * s2) / sd;
          if (rd_dx) v += PF ? cd[i] : add[r * ldadd + j];
          dr[j] = v;
        }
      }
    }
    if constexpr (PF) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        cx[i] = nx[i];
        cg[i] = ng[i];
        cd[i] = nd[i];
      }
    }
  }
  // waves 4..7 hand their sums to waves 0..3, then waves 1..3 to wave 0
  if (w >= 4) {
    float* rw = red + (int64_t)(w - 4) * 2 * C;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < C) {
        rw[j] = ag[i];
        rw[C + j] = ab[i];
      }
    }
  }
  __syncthreads();
  if (w < 4) {
    const float* rw = red + (int64_t)w * 2 * C;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < C) {
        ag[i] += rw[j];
        ab[i] += rw[C + j];
      }
    }
  }
  __syncthreads();
  if (w >= 1 && w < 4) {
    float* rw = red + (int64_t)(w - 1) * 2 * C;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < C) {
        rw[j] = ag[i];
        rw[C + j] = ab[i];
      }
    }
  }
  __syncthreads();
  if (w == 0) {
    float* out = ws + (int64_t)blockIdx.x * 2 * C;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int j = lane + 64 * i;
      if (j < C) {
        out[j] = ((ag[i] + red[j]) + red[2 * C + j]) + red[4 * C + j];
        out[C + j] = ((ab[i] + red[C + j]) + red[3 * C + j]) + red[5 * C + j];
      }
    }
  }
}

// dgamma / dbeta = sums of the nsplit block partials [s][2][C], in block
// order.  Block = 16 columns x 16 partial lanes; blockIdx.y picks dgamma (0)
// or dbeta (1).
__global__ __launch_bounds__(256) void layernorm_param_combine(const float* __restrict__ ws, int nsplit, int C,
                                                               float* __restrict__ dgamma,
                                                               float* __restrict__ dbeta, int accumulate) {
  __shared__ float part[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + tx;
  const int which = blockIdx.y;
  float a = 0.f;
  if (c < C) {
#pragma unroll 8
    for (int s = ty; s < nsplit; s += 16) a += ws[((int64_t)s * 2 + which) * C + c];
  }
  part[ty][tx] = a;
  __syncthreads();
  if (ty == 0 && c < C) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += part[k][tx];
    float* o = which ? dbeta : dgamma;
    if (accumulate) t += o[c];
    o[c] = t;
  }
}

// Row blocks of the fused backward: about 32 rows each (4 per wave), at most
// 1024 blocks (eight waves per SIMD on 256 CUs).
static int64_t ln_param_blocks(int64_t rows) {
  int64_t nb = (rows + 31) / 32;
  return nb < 1 ? 1 : (nb > 1024 ? 1024 : nb);
}

__global__ __launch_bounds__(256) void gelu_fwd_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    y[i] = gelu_tanh(x[i]);
  }
}

__global__ __launch_bounds__(256) void gelu_bwd_kernel(const float* __restrict__ x, const float* __restrict__ dy,
                                                       float* __restrict__ dx, int64_t n, int accumulate) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float r = gelu_grad(x[i]) * dy[i];
    if (accumulate) r += dx[i];
    dx[i] = r;
  }
}

// Cross-entropy forward: per-row loss_i = lse_i - x[i, y_i]; lse saved.
__global__ __launch_bounds__(256) void xent_fwd_kernel(const float* __restrict__ x, int64_t ldx,
                                                       const int64_t* __restrict__ labels,
                                                       float* __restrict__ row_loss, float* __restrict__ lse_out,
                                                       int64_t rows, int V) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * ldx;
  float mx = -INFINITY;
  for (int j = lane; j < V; j += 64) mx = fmaxf(mx, xr[j]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int j = lane; j < V; j += 64) s += expf(xr[j] - mx);
  s = wave_sum(s);
  if (lane == 0) {
    const float lse = mx + logf(s);
    int64_t y = labels[row];
    y = y < 0 ? 0 : (y >= V ? V - 1 : y);  // labels are validated on the host
    row_loss[row] = lse - xr[y];
    lse_out[row] = lse;
  }
}

// dx[i,j] = g * (exp(x[i,j] - lse_i) - [j == y_i]) * scale, g read from device
__global__ __launch_bounds__(256) void xent_bwd_kernel(const float* __restrict__ x, int64_t ldx,
                                                       const int64_t* __restrict__ labels,
                                                       const float* __restrict__ lse,
                                                       const float* __restrict__ gscalar, float scale,
                                                       float* __restrict__ dx, int64_t lddx, int64_t rows, int V,
                                                       int accumulate) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float g = gscalar[0] * scale;
  const float l = lse[row];
  const int64_t y = labels[row];
  const float* xr = x + row * ldx;
  float* dr = dx + row * lddx;
  for (int j = lane; j < V; j += 64) {
    float v = g * (expf(xr[j] - l) - (j == y ? 1.0f : 0.0f));
    if (accumulate) v += dr[j];
    dr[j] = v;
  }
}

int rows_grid(int64_t rows) { return (int)((rows + 3) / 4); }

template <template <int> class K>
struct Dummy {};

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_softmax_fwd_f32(const float* x, int64_t ldx, float* y, int64_t ldy, int64_t rows, int L,
                                   int causal_tq, int log_mode, void* stream) {
  MTX_CHECK_ARG(x && y, "softmax: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && L >= 1 && ldx >= L && ldy >= L, "softmax: bad rows/L/ld");
  MTX_CHECK_SHAPE(causal_tq >= 0 && causal_tq <= L, "softmax: causal_tq must be in [0, L]");
  if (rows == 0) return MTX_OK;
  MTX_CHECK_SHAPE(rows / 4 < (1LL << 31), "softmax: too many rows");
  hipLaunchKernelGGL(softmax_fwd_kernel, dim3(rows_grid(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     x, ldx, y, ldy, rows, L, causal_tq, log_mode ? 1 : 0);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_softmax_bwd_f32(const float* y, int64_t ldy, const float* dy, int64_t lddy, float* dx,
                                   int64_t lddx, int64_t rows, int L, int log_mode, int accumulate, void* stream) {
  MTX_CHECK_ARG(y && dy && dx, "softmax_bwd: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && L >= 1 && ldy >= L && lddy >= L && lddx >= L, "softmax_bwd: bad rows/L/ld");
  if (rows == 0) return MTX_OK;
  hipLaunchKernelGGL(softmax_bwd_kernel, dim3(rows_grid(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     y, ldy, dy, lddy, dx, lddx, rows, L, log_mode ? 1 : 0, accumulate ? 1 : 0);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_layernorm_fwd_f32(const float* x, int64_t ldx, const float* gamma, const float* beta,
                                     float* y, int64_t ldy, float* mean, float* std_, int64_t rows, int C,
                                     float eps, void* stream) {
  MTX_CHECK_ARG(x && gamma && beta && y && mean && std_, "layernorm: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && C >= 1 && C <= 64 * 32 && ldx >= C && ldy >= C,
                  "layernorm: C must be in [1, 2048] and ld >= C");
  if (rows == 0) return MTX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpl = (C + 63) / 64;
  dim3 gr(rows_grid(rows)), bl(256);
#define LN_F(V) hipLaunchKernelGGL(layernorm_fwd_kernel<V>, gr, bl, 0, st, x, ldx, gamma, beta, y, ldy, mean, std_, rows, C, eps)
  if (vpl <= 1) LN_F(1);
  else if (vpl <= 2) LN_F(2);
  else if (vpl <= 4) LN_F(4);
  else if (vpl <= 6) LN_F(6);
  else if (vpl <= 8) LN_F(8);
  else if (vpl <= 12) LN_F(12);
  else if (vpl <= 16) LN_F(16);
  else LN_F(32);
#undef LN_F
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" size_t mtx_layernorm_bwd_workspace_bytes(int64_t rows, int C) {
  if (rows < 1 || C < 1) return 0;
  return (size_t)ln_param_blocks(rows) * 2 * C * sizeof(float);
}

extern "C" int mtx_layernorm_bwd_f32(const float* x, int64_t ldx, const float* gamma, const float* mean,
                                     const float* std_, const float* dy, int64_t lddy, float* dx, int64_t lddx,
                                     const float* addend, int64_t ldadd, float* dgamma, float* dbeta, int64_t rows,
                                     int C, int accumulate, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  MTX_CHECK_ARG(x && gamma && mean && std_ && dy, "layernorm_bwd: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && C >= 1 && C <= 2048 && ldx >= C && lddy >= C, "layernorm_bwd: bad shape");
  MTX_CHECK_ARG(!dx || lddx >= C, "layernorm_bwd: bad lddx");
  MTX_CHECK_ARG((dgamma == nullptr) == (dbeta == nullptr), "layernorm_bwd: dgamma and dbeta go together");
  MTX_CHECK_ARG(accumulate >= 0 && accumulate <= 3, "layernorm_bwd: accumulate takes bits 0 (dx) and 1 (params)");
  MTX_CHECK_ARG(!addend || (dx && !(accumulate & 1) && ldadd >= C),
                "layernorm_bwd: an addend needs dx, no dx accumulation and ldadd >= C");
  if (rows == 0) return MTX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpl = (C + 63) / 64;
  const int acc_p = (accumulate >> 1) & 1;
  // accumulating into dx is dx = dx_ln + dx: the addend read from dx itself
  const float* add = (accumulate & 1) ? dx : addend;
  const int64_t lda = (accumulate & 1) ? lddx : ldadd;
  if (dgamma) {
    const size_t need = mtx_layernorm_bwd_workspace_bytes(rows, C);
    MTX_CHECK_ARG(workspace && workspace_bytes >= need, "layernorm_bwd: workspace too small (%zu < %zu)",
                  workspace_bytes, need);
    const int nsplit = (int)ln_param_blocks(rows);
    const int64_t chunk = (rows + nsplit - 1) / nsplit;
    float* ws = static_cast<float*>(workspace);
    const size_t lds = (size_t)8 * C * sizeof(float);
#define LN_P(V) hipLaunchKernelGGL(layernorm_bwd_param_kernel<V>, dim3(nsplit), dim3(64 * LNP_WAVES), lds, st, x, ldx, gamma, mean, std_, dy, lddy, dx, lddx, add, lda, ws, rows, C, chunk)
    if (vpl <= 1) LN_P(1);
    else if (vpl <= 2) LN_P(2);
    else if (vpl <= 4) LN_P(4);
    else if (vpl <= 6) LN_P(6);
    else if (vpl <= 8) LN_P(8);
    else if (vpl <= 12) LN_P(12);
    else if (vpl <= 16) LN_P(16);
    else LN_P(32);
#undef LN_P
    MTX_LAUNCHED();
    hipLaunchKernelGGL(layernorm_param_combine, dim3((C + 15) / 16, 2), dim3(256), 0, st, ws, nsplit, C, dgamma,
                       dbeta, acc_p);
    MTX_LAUNCHED();
  } else if (dx) {
    dim3 gr(rows_grid(rows)), bl(256);
#define LN_B(V) hipLaunchKernelGGL(layernorm_bwd_kernel<V>, gr, bl, 0, st, x, ldx, gamma, mean, std_, dy, lddy, dx, lddx, add, lda, rows, C)
    if (vpl <= 1) LN_B(1);
    else if (vpl <= 2) LN_B(2);
    else if (vpl <= 4) LN_B(4);
    else if (vpl <= 6) LN_B(6);
    else if (vpl <= 8) LN_B(8);
    else if (vpl <= 12) LN_B(12);
    else if (vpl <= 16) LN_B(16);
    else LN_B(32);
#undef LN_B
    MTX_LAUNCHED();
  }
  return MTX_OK;
}

extern "C" int mtx_gelu_fwd_f32(const float* x, float* y, int64_t n, void* stream) {
  MTX_CHECK_ARG(x && y && n >= 0, "gelu: bad argument");
  if (n == 0) return MTX_OK;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 16384);
  hipLaunchKernelGGL(gelu_fwd_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, y, n);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_gelu_bwd_f32(const float* x, const float* dy, float* dx, int64_t n, int accumulate,
                                void* stream) {
  MTX_CHECK_ARG(x && dy && dx && n >= 0, "gelu_bwd: bad argument");
  if (n == 0) return MTX_OK;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 16384);
  hipLaunchKernelGGL(gelu_bwd_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, dy, dx, n,
                     accumulate ? 1 : 0);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_xent_fwd_f32(const float* logits, int64_t ld, const int64_t* labels, float* row_loss,
                                float* lse, int64_t rows, int V, void* stream) {
  MTX_CHECK_ARG(logits && labels && row_loss && lse, "xent: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && V >= 1 && ld >= V, "xent: bad shape");
  if (rows == 0) return MTX_OK;
  hipLaunchKernelGGL(xent_fwd_kernel, dim3(rows_grid(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     logits, ld, labels, row_loss, lse, rows, V);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_xent_bwd_f32(const float* logits, int64_t ld, const int64_t* labels, const float* lse,
                                const float* gscalar, float scale, float* dlogits, int64_t ldd, int64_t rows, int V,
                                int accumulate, void* stream) {
  MTX_CHECK_ARG(logits && labels && lse && gscalar && dlogits, "xent_bwd: null pointer");
  MTX_CHECK_SHAPE(rows >= 0 && V >= 1 && ld >= V && ldd >= V, "xent_bwd: bad shape");
  if (rows == 0) return MTX_OK;
  hipLaunchKernelGGL(xent_bwd_kernel, dim3(rows_grid(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     logits, ld, labels, lse, gscalar, scale, dlogits, ldd, rows, V, accumulate ? 1 : 0);
  MTX_LAUNCHED();
  return MTX_OK;
}
