// Decode-time attention (one new query per sequence against its cached keys)
// and the device-side greedy pick, for gfx950 (MI355X).
//
// mtx_attn_decode replaces, for the incremental step of generation, the
// reference's attention sub-graph (transformer.py:36-44) evaluated at the last
// position: o = softmax(scale * q k^T) v over the L cached keys.  The
// reference recomputes the whole forward per token (GPT.generate,
// transformer.py:93-104); with a KV cache the step's attention is this
// product, which reads K and V once and is HBM / cache bound.
//
// One workgroup per (b, h):
//   phase 1: thread t owns keys t, t+256, ...; it reads the key row (D
//            contiguous elements) and forms s = (c q).k in registers, where
//            c = scale*log2(e); scores go to LDS, the max and the sum of
//            exp2(s - max) are reduced over the workgroup;
//   phase 2: thread t owns output elements 4*(t % (D/4)) .. +3 for the key
//            group t / (D/4); a value row per key is read by D/4 adjacent
//            threads (coalesced), several keys in flight per thread, and the
//            key groups are summed through LDS.
// mtx_argmax_f32 is np.argmax over rows (first maximum) plus the top-2 margin,
// the greedy harness's pick, so decoding needs no host round trip per token.
// mtx_kv_append_f32 and mtx_decode_advance keep a decode step's positions in
// device memory, so one recorded step (a HIP graph) replays for every token.
#include "mtx_common.h"
#include "decode_pick.h"

#include <algorithm>
#include <cmath>

namespace mtx {
namespace {

constexpr int kDecThreads = 256;
constexpr int kDecMaxL = 8192;  // scores held in LDS: 32 KiB

struct DecStr {
  int64_t b, h, t;  // element strides; the d stride is 1
};

struct DecArgs {
  const void* q; DecStr sq;
  const void* k; DecStr sk;
  const void* v; DecStr sv;
  void* o; DecStr so;
  float* lse;
  const int* lengths;
  int B, H, L;
  float scale;
};

template <typename T, int E>
__device__ __forceinline__ void load_row(const T* __restrict__ p, float* out) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < E; e += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + e);
      out[e] = v[0]; out[e + 1] = v[1]; out[e + 2] = v[2]; out[e + 3] = v[3];
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; e += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + e);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[e + 2 * i] = __uint_as_float(w[i] << 16);
        out[e + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    }
  }
}

template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xffff0000u)};
  }
}

template <typename T>
__device__ __forceinline__ void store1(T* p, float x) {
  if constexpr (sizeof(T) == 4) *p = x;
  else *p = f2bf(x);
}

template <typename T, int D>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(const DecArgs a) {
  extern __shared__ float smem[];  // [L] scores, then reduction scratch
  __shared__ float red[kDecThreads / 64];
  __shared__ __attribute__((aligned(16))) float part[kDecThreads * 4];

  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int L = a.L;
  if (a.lengths != nullptr) L = min(max(a.lengths[b], 0), a.L);
  const T* __restrict__ qp = static_cast<const T*>(a.q) + b * a.sq.b + h * a.sq.h;
  const T* __restrict__ kp = static_cast<const T*>(a.k) + b * a.sk.b + h * a.sk.h;
  const T* __restrict__ vp = static_cast<const T*>(a.v) + b * a.sv.b + h * a.sv.h;
  T* __restrict__ op = static_cast<T*>(a.o) + b * a.so.b + h * a.so.h;
  const float c = a.scale * kLog2e;

  // ---- phase 1: scores (log2 units) ----
  float q[D];
  load_row<T, D>(qp, q);
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] *= c;
  float mx = -INFINITY;
  for (int j = tid; j < L; j += kDecThreads) {
    const T* __restrict__ kr = kp + (int64_t)j * a.sk.t;
    float s = 0.f;
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 16) {
      float kc[16];
      load_row<T, 16>(kr + d0, kc);
#pragma unroll
      for (int e = 0; e < 16; ++e) s = fmaf(q[d0 + e], kc[e], s);
    }
    smem[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wid] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
  for (int j = tid; j < L; j += kDecThreads) {
    const float p = __builtin_amdgcn_exp2f(smem[j] - mx);
    smem[j] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[wid] = sum;
  __syncthreads();  // also publishes every p_j
  const float l = (red[0] + red[1]) + (red[2] + red[3]);

  // ---- phase 2: o[d] = sum_j p_j v[j][d] / l ----
  constexpr int DV = D / 4;             // 4-element slices per row
  constexpr int NG = kDecThreads / DV;  // key groups
  const int dv = tid % DV, kg = tid / DV;
  f32x4 acc = zero4();
#pragma unroll 4
  for (int j = kg; j < L; j += NG) acc += smem[j] * load4<T>(vp + (int64_t)j * a.sv.t + 4 * dv);
  *reinterpret_cast<f32x4*>(part + kg * D + 4 * dv) = acc;
  __syncthreads();
  if (tid < D) {
    float o = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) o += part[g * D + tid];
    store1<T>(op + tid, L > 0 ? o / l : 0.f);
    if (tid == 0 && a.lse != nullptr) a.lse[bh] = L > 0 ? (mx + __log2f(l)) * kLn2 : -INFINITY;
  }
}

// ---- a decode step's q/k/v projection and attention in one launch (fp32) ----
// One workgroup of kQaW waves per head h and group of S sequences.  It forms
// the group's q, k and v rows of head h from the step's (normalised) input
// rows x[b] and the packed (C, 3C) projection (each wave a range of C, the
// wave sums added in wave order, then the bias), writes k and v to cache row
// lengths[b] - 1, and runs the attention of mtx_attn_decode over the first
// lengths[b] cached rows, kQaW / S waves per sequence, taking the new row from
// LDS (the cache write is not read back).  Each weight element is loaded once
// per group: the workgroups of a head share the 3 x C x D slab through the
// XCD's L2, so S sequences per workgroup divide that traffic by S.
#ifndef MTX_QA_WAVES
#define MTX_QA_WAVES 16
#endif
#ifndef MTX_QA_SEQ
#define MTX_QA_SEQ 2
#endif
constexpr int kQaW = MTX_QA_WAVES;
constexpr int kQaThreads = 64 * kQaW;
constexpr int kQaS = MTX_QA_SEQ;  // sequences per workgroup for D = 64 (D = 128: 1)
constexpr int kQaMaxC = 1024;
constexpr int kQaMaxT = 2048;      // scores of S sequences in dynamic LDS

// A decode step's input rows given raw: r = x[b], plus, with pending partial
// products pws (pks of them, [pks][B][C]), r = (sum_s pws[s][b] + pbias) + r,
// the arithmetic of splitk_reduce_ln_kernel with alpha = beta = 1 (written to
// x_out[b] when x_out is set); the kernel then reads the LayerNorm of r
// (gamma, beta, eps; C <= 1024).
struct PendingLn {
  const float* pws;
  int pks;
  const float* pbias;
  float* x_out;
  int64_t ldxo;
  const float* gamma;
  const float* beta;
  float eps;
};

// element n of row b of the updated residual: x[b][n] or, with pending
// partial products, (sum_s pws[s][b][n] + pbias[n]) + x[b][n]; the pks <= 8
// loads are independent (indices clamped, the unused ones discarded)
__device__ __forceinline__ float pending_elem(const PendingLn& pl, const float* __restrict__ x, int64_t ldx, int B,
                                              int C, int b, int n) {
  const float r = x[(int64_t)b * ldx + n];
  if (!pl.pws) return r;
  float pv[8];
#pragma unroll
  for (int sp = 0; sp < 8; ++sp) pv[sp] = pl.pws[((int64_t)min(sp, pl.pks - 1) * B + b) * C + n];
  float s = 0.f;
#pragma unroll
  for (int sp = 0; sp < 8; ++sp)
    if (sp < pl.pks) s += pv[sp];
  float t = s + (pl.pbias ? pl.pbias[n] : 0.f);
  t += r;
  return t;
}

// LayerNorm of one LDS row of C <= 1024 values by one wave, in place
__device__ __forceinline__ void ln_row_lds(float* __restrict__ row, int C, int lane, const PendingLn& pl) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int n = lane + 64 * i;
    v[i] = n < C ? row[n] : 0.f;
  }
  float mean, sd;
  ln_stats<16>(v, lane, C, pl.eps, mean, sd);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int n = lane + 64 * i;
    if (n < C) row[n] = ln_apply(v[i], sd, pl.gamma[n], pl.beta[n]);
  }
}

template <int D, int S>
__global__ __launch_bounds__(kQaThreads) void qkv_attn_kernel(int B, int H, int C, const float* __restrict__ x,
                                                              int64_t ldx, const PendingLn pl,
                                                              const float* __restrict__ W, int64_t ldw,
                                                              const float* __restrict__ bias, float* __restrict__ kc,
                                                              float* __restrict__ vc, int64_t csb, int64_t cst,
                                                              int Tmax, const int* __restrict__ lengths, float scale,
                                                              float* __restrict__ o, int64_t ldo) {
  constexpr int NC = 3 * D;     // head h's q, k and v columns
  constexpr int NPL = NC / 64;  // of which each lane owns NPL
  constexpr int WS = kQaW / S;  // waves per sequence in the attention
  constexpr int TPS = 64 * WS;
  constexpr int DV = D / 4, NGS = TPS / DV;  // value slices, key groups per sequence
  constexpr int GPF = kQaW * S * NC;          // wave partial sums
  constexpr int PTF = S * NGS * D;            // key-group partial outputs
  static_assert(kQaW % S == 0 && NPL * 64 == NC, "workgroup shape");
  extern __shared__ float sc[];                                     // [S][Tmax] scores
  __shared__ __attribute__((aligned(16))) float xs[S][kQaMaxC];
  __shared__ __attribute__((aligned(16))) float buf[GPF > PTF ? GPF : PTF];  // wave sums, then key groups
  __shared__ __attribute__((aligned(16))) float qkv[S][NC];
  __shared__ float red[kQaW];

  const int b0 = (blockIdx.x / H) * S, h = blockIdx.x % H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  // q, k, v: wave w sums over rows [k0, k1) of the weight, in batches of kB
  // rows whose loads are all issued before their products; the first batch
  // is requested before the input rows are read, so both latencies overlap
  int64_t col[NPL];
#pragma unroll
  for (int t = 0; t < NPL; ++t) {
    const int jj = lane + 64 * t;
    col[t] = (int64_t)(jj / D) * C + h * D + jj % D;
  }
  const int kcnt = (C + kQaW - 1) / kQaW;
  const int k0 = w * kcnt, k1 = min(C, k0 + kcnt);
  constexpr int kB = (NPL >= 6 ? 60 : 72) / NPL;
  float wv[kB][NPL];
  auto load_batch = [&](int kb) {
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int64_t r = min(kb + j, C - 1);
#pragma unroll
      for (int t = 0; t < NPL; ++t) wv[j][t] = W[r * ldw + col[t]];
    }
  };
  load_batch(k0);

  if (pl.gamma) {
    // raw rows (plus pending partial products), one element per thread; the
    // head-0 workgroup of the group writes the updated rows; then wave s
    // normalises row s
    for (int i = tid; i < S * C; i += kQaThreads) {
      const int s = i / C, n = i % C;
      float t = 0.f;
      if (b0 + s < B) {
        t = pending_elem(pl, x, ldx, B, C, b0 + s, n);
        if (h == 0 && pl.x_out) pl.x_out[(int64_t)(b0 + s) * pl.ldxo + n] = t;
      }
      xs[s][n] = t;
    }
    __syncthreads();
    if (w < S) ln_row_lds(xs[w], C, lane, pl);
  } else {
    for (int i = tid; i < S * C; i += kQaThreads) {
      const int s = i / C, k = i % C;
      xs[s][k] = b0 + s < B ? x[(int64_t)(b0 + s) * ldx + k] : 0.f;
    }
  }
  __syncthreads();

  float acc[S][NPL];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < NPL; ++t) acc[s][t] = 0.f;
  for (int kb = k0; kb < k1; kb += kB) {
    if (kb != k0) load_batch(kb);
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (kb + j < k1) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const float xv = xs[s][kb + j];
#pragma unroll
          for (int t = 0; t < NPL; ++t) acc[s][t] = fmaf(xv, wv[j][t], acc[s][t]);
        }
      }
    }
  }
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < NPL; ++t) buf[(w * S + s) * NC + lane + 64 * t] = acc[s][t];
  __syncthreads();
  for (int i = tid; i < S * NC; i += kQaThreads) {
    const int s = i / NC, jj = i % NC;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kQaW; ++q) v += buf[(q * S + s) * NC + jj];
    const int pt = jj / D, e = jj % D;
    if (bias) v += bias[pt * C + h * D + e];
    qkv[s][jj] = v;
    const int b = b0 + s;
    if (pt > 0 && b < B) {
      const int t = lengths[b] - 1;
      if (t >= 0 && t < Tmax) (pt == 1 ? kc : vc)[(int64_t)b * csb + (int64_t)t * cst + h * D + e] = v;
    }
  }
  __syncthreads();

  // ---- attention: waves [sg*WS, sg*WS + WS) take sequence b0 + sg ----
  const int sg = w / WS, lt = tid % TPS;
  const int b = b0 + sg;
  const int len = b < B ? lengths[b] : 0;
  const int L = min(max(len, 0), Tmax);
  const int newrow = (len >= 1 && len <= Tmax) ? len - 1 : -1;  // the row this step wrote
  float* __restrict__ scs = sc + sg * Tmax;
  const float* __restrict__ qv = qkv[sg];
  // scores (log2 units): four threads per key, a quarter of D each
  const float c = scale * kLog2e;
  constexpr int DQ = D / 4;
  const int kq = lt >> 2, qd = lt & 3;
  float qr[DQ];
#pragma unroll
  for (int e = 0; e < DQ; ++e) qr[e] = qv[qd * DQ + e] * c;
  const float* __restrict__ kb0 = kc + (int64_t)min(b, B - 1) * csb + h * D + qd * DQ;
  float mx = -INFINITY;
  for (int j = kq; j < L; j += TPS / 4) {
    float kr[DQ];
    if (j == newrow) {
#pragma unroll
      for (int e = 0; e < DQ; ++e) kr[e] = qv[D + qd * DQ + e];
    } else {
#pragma unroll
      for (int e = 0; e < DQ; e += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(kb0 + (int64_t)j * cst + e);
        kr[e] = v[0]; kr[e + 1] = v[1]; kr[e + 2] = v[2]; kr[e + 3] = v[3];
      }
    }
    float sv = 0.f;
#pragma unroll
    for (int e = 0; e < DQ; ++e) sv = fmaf(qr[e], kr[e], sv);
    sv += __shfl_xor(sv, 1, 64);
    sv += __shfl_xor(sv, 2, 64);
    if (qd == 0) scs[j] = sv;
    mx = fmaxf(mx, sv);
  }
  mx = wave_max(mx);
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = red[sg * WS];
#pragma unroll
  for (int q = 1; q < WS; ++q) mx = fmaxf(mx, red[sg * WS + q]);
  __syncthreads();
  float sum = 0.f;
  for (int j = lt; j < L; j += TPS) {
    const float p = __builtin_amdgcn_exp2f(scs[j] - mx);
    scs[j] = p;
    sum += p;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[w] = sum;
  __syncthreads();  // also publishes every p_j
  float l = 0.f;
#pragma unroll
  for (int q = 0; q < WS; ++q) l += red[sg * WS + q];

  // o[d] = sum_j p_j v[j][d] / l
  const int dv = lt % DV, kg = lt / DV;
  const float* __restrict__ vb0 = vc + (int64_t)min(b, B - 1) * csb + h * D + 4 * dv;
  f32x4 av = zero4();
#pragma unroll 4
  for (int j = kg; j < L; j += NGS) {
    const f32x4 vv = j == newrow ? *reinterpret_cast<const f32x4*>(qv + 2 * D + 4 * dv)
                                 : *reinterpret_cast<const f32x4*>(vb0 + (int64_t)j * cst);
    av += scs[j] * vv;
  }
  *reinterpret_cast<f32x4*>(buf + (sg * NGS + kg) * D + 4 * dv) = av;
  __syncthreads();
  if (lt < D && b < B) {
    float r = 0.f;
#pragma unroll 8
    for (int g = 0; g < NGS; ++g) r += buf[(sg * NGS + g) * D + lt];
    o[(int64_t)b * ldo + h * D + lt] = L > 0 ? r / l : 0.f;
  }
}

__global__ __launch_bounds__(256) void argmax_kernel(int rows, int cols, const float* __restrict__ x,
                                                     int64_t ld, int64_t* __restrict__ idx, int64_t idx_stride,
                                                     float* __restrict__ margin, int64_t margin_stride) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // wave-uniform
  const float* __restrict__ xr = x + (int64_t)row * ld;
  Top2 t{-INFINITY, -INFINITY, cols};
  for (int c = lane; c < cols; c += 64) scan(t, xr[c], c, cols);
  t = reduce_top2(t, cols);
  if (lane == 0) {
    idx[(int64_t)row * idx_stride] = t.i1;
    if (margin != nullptr) margin[(int64_t)row * margin_stride] = t.m1 - t.m2;
  }
}

// cache[b, lengths[b] - 1, :] = x[b, :] (rows outside [0, T) are skipped)
__global__ __launch_bounds__(256) void kv_append_kernel(int B, int C, int T, const float* __restrict__ x,
                                                        int64_t sxb, float* __restrict__ cache, int64_t scb,
                                                        int64_t sct, const int* __restrict__ lengths) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)B * C) return;
  const int b = (int)(i / C), c = (int)(i % C);
  const int t = lengths[b] - 1;
  if (t < 0 || t >= T) return;
  cache[b * scb + (int64_t)t * sct + c] = x[b * sxb + c];
}

// lengths[b] += 1 for every b; pos[0] += 1
// The greedy step's pick, record and bookkeeping in one launch: row b's
// first-maximum index goes to cur[b] (the next step's input) and to the
// time-major id buffer at row lengths[b] (the position the token takes), the
// top-2 margin to margins at row lengths[b] - t_base, then lengths[b] += 1;
// row 0 also advances the position id.  Each row's lengths entry is read and
// written by that row's lane 0 only.
__global__ __launch_bounds__(256) void greedy_pick_kernel(int rows, int cols, const float* __restrict__ x,
                                                          int64_t ld, int64_t* __restrict__ cur,
                                                          int64_t* __restrict__ ids, int Tmax,
                                                          float* __restrict__ margins, int t_base, int nm,
                                                          int* __restrict__ lengths, int64_t* __restrict__ pos) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;  // wave-uniform
  const float* __restrict__ xr = x + (int64_t)row * ld;
  Top2 t{-INFINITY, -INFINITY, cols};
  for (int c = lane; c < cols; c += 64) scan(t, xr[c], c, cols);
  t = reduce_top2(t, cols);
  if (lane == 0) {
    const int L = lengths[row];
    cur[row] = t.i1;
    if (L >= 0 && L < Tmax) ids[(int64_t)L * rows + row] = t.i1;
    const int s = L - t_base;
    if (margins != nullptr && s >= 0 && s < nm) margins[(int64_t)s * rows + row] = t.m1 - t.m2;
    lengths[row] = L + 1;
    if (row == 0 && pos != nullptr) pos[0] += 1;
  }
}

// out[i] = wa[ia[i]] + wb[ib[i * ib_stride]]: the token and position
// embeddings and their sum (transformer.py:84-87) in one pass; ids are
// clamped to the tables (they are validated on the host)
__global__ __launch_bounds__(256) void embed2_kernel(const float* __restrict__ wa, int64_t lda, int64_t Va,
                                                     const int64_t* __restrict__ ia,
                                                     const float* __restrict__ wb, int64_t ldb, int64_t Vb,
                                                     const int64_t* __restrict__ ib, int64_t ib_stride,
                                                     float* __restrict__ out, int64_t ldo, int64_t n, int C) {
  const int64_t total = n * C;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / C;
    const int c = (int)(e % C);
    int64_t ra = ia[i], rb = ib[i * ib_stride];
    ra = ra < 0 ? 0 : (ra >= Va ? Va - 1 : ra);
    rb = rb < 0 ? 0 : (rb >= Vb ? Vb - 1 : rb);
    out[i * ldo + c] = wa[ra * lda + c] + wb[rb * ldb + c];
  }
}


// The output projection and the greedy pick of one decode step in one
// launch: one 16-wave workgroup per row.  Wave w sums the K range
// [w * kc, (w + 1) * kc) for the lane's logits j, j + 64, ... (x's row staged
// in LDS and read as a broadcast, one fused multiply-add per term, k
// ascending), the 16 partial sums are added in wave order with the bias,
// then the top two over the row and the pick's bookkeeping as
// greedy_pick_kernel.
constexpr int kHpW = 16;  // waves per head_pick workgroup
template <int VPL>
__global__ __launch_bounds__(64 * kHpW) void head_pick_kernel(int rows, int K, int V, const float* __restrict__ x,
                                                              int64_t ldx, const PendingLn pl,
                                                              const float* __restrict__ W, int64_t ldw,
                                                              const float* __restrict__ bias,
                                                              int64_t* __restrict__ cur, int64_t* __restrict__ ids,
                                                              int Tmax, float* __restrict__ margins, int t_base,
                                                              int nm, int* __restrict__ lengths,
                                                              int64_t* __restrict__ pos) {
  extern __shared__ float smem[];
  float* xs = smem;                       // K floats
  float* part = smem + ((K + 3) & ~3);    // kHpW x 64 * VPL partial sums
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // the weight rows of the wave's K range in batches of kHpB, every load of
  // a batch issued before its products; the first batch is requested before
  // the input row is read, so both latencies overlap
  const int kc = (K + kHpW - 1) / kHpW;
  const int k0 = w * kc, k1 = min(K, k0 + kc);
  constexpr int kHpB = VPL == 1 ? 32 : 48 / VPL;
  float wv[kHpB][VPL];
  auto load_batch = [&](int kb) {
#pragma unroll
    for (int j = 0; j < kHpB; ++j) {
      const int k = min(kb + j, K - 1);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = min(lane + 64 * i, V - 1);
        wv[j][i] = W[(int64_t)k * ldw + c];
      }
    }
  };
  load_batch(k0);
  if (pl.gamma) {
    // the raw row (plus pending partial products), one element per thread,
    // normalised by wave 0
    for (int n = tid; n < K; n += 64 * kHpW) xs[n] = pending_elem(pl, x, ldx, rows, K, row, n);
    __syncthreads();
    if (w == 0) ln_row_lds(xs, K, lane, pl);
  } else {
    const float* __restrict__ xr = x + (int64_t)row * ldx;
    for (int k = tid; k < K; k += 64 * kHpW) xs[k] = xr[k];
  }
  __syncthreads();
  float acc[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) acc[i] = 0.f;
  for (int kb = k0; kb < k1; kb += kHpB) {
    if (kb != k0) load_batch(kb);
#pragma unroll
    for (int j = 0; j < kHpB; ++j) {
      if (kb + j < k1) {
        const float xv = xs[kb + j];
#pragma unroll
        for (int i = 0; i < VPL; ++i) acc[i] = fmaf(xv, wv[j][i], acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) part[w * 64 * VPL + lane + 64 * i] = acc[i];
  __syncthreads();
  if (w != 0) return;
  Top2 t{-INFINITY, -INFINITY, V};
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < V) {
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < kHpW; ++q) v += part[q * 64 * VPL + c];
      if (bias) v += bias[c];
      scan(t, v, c, V);
    }
  }
  t = reduce_top2(t, V);
  if (lane == 0) pick_record(row, rows, t, cur, ids, Tmax, margins, t_base, nm, lengths, pos);
}

// The token and position embeddings, their sum, and the first block's
// LayerNorm of it in one launch: one wave per row, the sum written to out
// and normalised into y (the arithmetic of embed2_kernel and
// layernorm_fwd_kernel).
template <int VPL>
__global__ __launch_bounds__(64) void embed2_ln_kernel(const float* __restrict__ wa, int64_t lda, int64_t Va,
                                                       const int64_t* __restrict__ ia,
                                                       const float* __restrict__ wb, int64_t ldb, int64_t Vb,
                                                       const int64_t* __restrict__ ib, int64_t ib_stride,
                                                       float* __restrict__ out, int64_t ldo, int C,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, float eps,
                                                       float* __restrict__ y, int64_t ldy) {
  const int64_t i = blockIdx.x;
  const int lane = threadIdx.x;
  int64_t ra = ia[i], rb = ib[i * ib_stride];
  ra = ra < 0 ? 0 : (ra >= Va ? Va - 1 : ra);
  rb = rb < 0 ? 0 : (rb >= Vb ? Vb - 1 : rb);
  float v[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < C ? wa[ra * lda + c] + wb[rb * ldb + c] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j;
    if (c < C) out[i * ldo + c] = v[j];
  }
  float mean, sd;
  ln_stats<VPL>(v, lane, C, eps, mean, sd);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int c = lane + 64 * j;
    if (c < C) y[i * ldy + c] = ln_apply(v[j], sd, gamma[c], beta[c]);
  }
}

__global__ void advance_kernel(int B, int* __restrict__ lengths, int64_t* __restrict__ pos) {
  const int i = threadIdx.x + blockIdx.x * blockDim.x;
  if (i < B) lengths[i] += 1;
  if (i == 0 && pos != nullptr) pos[0] += 1;
}

int check_row3(const char* name, const void* p, const int64_t* s, int esize) {
  MTX_CHECK_ARG(p != nullptr, "%s: null pointer", name);
  MTX_CHECK_ARG(s != nullptr, "%s: null strides", name);
  MTX_CHECK_ARG(s[3] == 1, "%s: the d stride must be 1 (got %lld)", name, (long long)s[3]);
  const int vec = 16 / esize;
  for (int i = 0; i < 3; ++i)
    MTX_CHECK_ARG(s[i] >= 0 && s[i] % vec == 0,
                  "%s: stride[%d]=%lld must be a non-negative multiple of %d elements", name, i,
                  (long long)s[i], vec);
  MTX_CHECK_ARG(((uintptr_t)p & 15u) == 0, "%s: pointer must be 16-byte aligned", name);
  return MTX_OK;
}

template <typename T, int D>
int launch_decode(const DecArgs& a, hipStream_t st) {
  const size_t lds = (size_t)(a.L > 0 ? a.L : 1) * sizeof(float);
  hipLaunchKernelGGL((attn_decode_kernel<T, D>), dim3(a.B * a.H), dim3(kDecThreads), lds, st, a);
  MTX_LAUNCHED();
  return MTX_OK;
}

template <typename T>
int dispatch_decode(int D, const DecArgs& a, hipStream_t st) {
  switch (D) {
    case 16: return launch_decode<T, 16>(a, st);
    case 32: return launch_decode<T, 32>(a, st);
    case 64: return launch_decode<T, 64>(a, st);
    default: return launch_decode<T, 128>(a, st);
  }
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_decode_qkv_attn_f32(int B, int H, int D, const float* x, int64_t ldx, const float* pws, int pks,
                                       const float* pbias, float* x_out, int64_t ldxo, const float* ln_gamma,
                                       const float* ln_beta, float eps, const float* W, int64_t ldw,
                                       const float* bias, float* kc, float* vc, int64_t csb, int64_t cst, int Tmax,
                                       const int* lengths, float scale, float* o, int64_t ldo, void* stream) {
  MTX_CHECK_ARG(x && W && kc && vc && lengths && o, "decode_qkv_attn: null pointer");
  MTX_CHECK_ARG(ln_gamma ? ln_beta != nullptr : (pws == nullptr && x_out == nullptr),
                "decode_qkv_attn: pending partials and x_out need the LayerNorm (gamma and beta)");
  MTX_CHECK_ARG(!pws || (pks >= 1 && pks <= 8), "decode_qkv_attn: 1 to 8 pending partial products");
  MTX_CHECK_ARG(!x_out || (ldxo >= (int64_t)H * D && (x_out >= x + (int64_t)(B - 1) * ldx + (int64_t)H * D ||
                                                       x >= x_out + (int64_t)(B - 1) * ldxo + (int64_t)H * D)),
                "decode_qkv_attn: x_out must hold H*D values per row and not overlap x");
  const int64_t C = (int64_t)H * D;
  MTX_CHECK_SHAPE(B >= 1 && H >= 1 && (D == 64 || D == 128) && C <= kQaMaxC && Tmax >= 1 && Tmax <= kQaMaxT,
                  "decode_qkv_attn: needs D in {64, 128}, H*D <= %d and 1 <= Tmax <= %d (got H=%d D=%d Tmax=%d)",
                  kQaMaxC, kQaMaxT, H, D, Tmax);
  MTX_CHECK_SHAPE(ldx >= C && ldw >= 3 * C && ldo >= C && cst >= C && csb >= (int64_t)Tmax * cst,
                  "decode_qkv_attn: bad strides");
  MTX_CHECK_ARG(cst % 4 == 0 && csb % 4 == 0 && ((uintptr_t)kc & 15u) == 0 && ((uintptr_t)vc & 15u) == 0,
                "decode_qkv_attn: cache rows must be 16-byte aligned");
  MTX_CHECK_ARG(std::isfinite(scale) && scale > 0.f, "scale must be finite and > 0");
  MTX_CHECK_ARG(std::isfinite(eps) && eps >= 0.f, "decode_qkv_attn: eps must be finite and >= 0");
  const PendingLn pl{pws, pks, pbias, x_out, ldxo, ln_gamma, ln_beta, eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (D == 64) {
    const size_t lds = (size_t)kQaS * Tmax * sizeof(float);
    hipLaunchKernelGGL((qkv_attn_kernel<64, kQaS>), dim3(((B + kQaS - 1) / kQaS) * H), dim3(kQaThreads), lds, st, B,
                       H, (int)C, x, ldx, pl, W, ldw, bias, kc, vc, csb, cst, Tmax, lengths, scale, o, ldo);
  } else {
    const size_t lds = (size_t)Tmax * sizeof(float);
    hipLaunchKernelGGL((qkv_attn_kernel<128, 1>), dim3(B * H), dim3(kQaThreads), lds, st, B, H, (int)C, x, ldx, pl,
                       W, ldw, bias, kc, vc, csb, cst, Tmax, lengths, scale, o, ldo);
  }
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_attn_decode(int dtype, int B, int H, int L, int D,
                               const void* q, const int64_t* q_strides,
                               const void* k, const int64_t* k_strides,
                               const void* v, const int64_t* v_strides,
                               void* o, const int64_t* o_strides,
                               float* lse, const int* lengths, float scale, void* stream) {
  if (dtype != MTX_F32 && dtype != MTX_BF16) return fail(MTX_ERR_DTYPE, "unsupported dtype %d", dtype);
  MTX_CHECK_SHAPE(B >= 1 && H >= 1 && (int64_t)B * H <= (1 << 24), "B,H must be >= 1 (got %d,%d)", B, H);
  MTX_CHECK_SHAPE(L >= 0 && L <= kDecMaxL, "decode needs 0 <= L <= %d cached keys (got %d)", kDecMaxL, L);
  MTX_CHECK_SHAPE(D == 16 || D == 32 || D == 64 || D == 128, "head dim D=%d not in {16,32,64,128}", D);
  const int es = dtype == MTX_F32 ? 4 : 2;
  int rc;
  if ((rc = check_row3("q", q, q_strides, es))) return rc;
  if ((rc = check_row3("k", k, k_strides, es))) return rc;
  if ((rc = check_row3("v", v, v_strides, es))) return rc;
  if ((rc = check_row3("o", o, o_strides, es))) return rc;
  MTX_CHECK_ARG(std::isfinite(scale) && scale > 0.f, "scale must be finite and > 0");
  DecArgs a{q, {q_strides[0], q_strides[1], q_strides[2]},
            k, {k_strides[0], k_strides[1], k_strides[2]},
            v, {v_strides[0], v_strides[1], v_strides[2]},
            o, {o_strides[0], o_strides[1], o_strides[2]},
            lse, lengths, B, H, L, scale};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == MTX_F32 ? dispatch_decode<float>(D, a, st) : dispatch_decode<bf16_t>(D, a, st);
}

extern "C" int mtx_argmax_f32(int rows, int cols, const float* x, int64_t ld, int64_t* idx,
                              int64_t idx_stride, float* margin, int64_t margin_stride, void* stream) {
  MTX_CHECK_SHAPE(rows >= 1 && cols >= 1, "rows, cols must be >= 1 (got %d, %d)", rows, cols);
  MTX_CHECK_ARG(x != nullptr && idx != nullptr, "x, idx: null pointer");
  MTX_CHECK_ARG(ld >= cols, "ld=%lld < cols=%d", (long long)ld, cols);
  hipLaunchKernelGGL(argmax_kernel, dim3((rows + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream),
                     rows, cols, x, ld, idx, idx_stride, margin, margin_stride);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_kv_append_f32(int B, int C, int T, const float* x, int64_t x_stride_b, float* cache,
                                 int64_t cache_stride_b, int64_t cache_stride_t, const int* lengths,
                                 void* stream) {
  MTX_CHECK_SHAPE(B >= 1 && C >= 1 && T >= 1, "B, C, T must be >= 1 (got %d, %d, %d)", B, C, T);
  MTX_CHECK_ARG(x != nullptr && cache != nullptr && lengths != nullptr, "x, cache, lengths: null pointer");
  MTX_CHECK_ARG(x_stride_b >= C && cache_stride_t >= C && cache_stride_b >= (int64_t)T * cache_stride_t,
                "strides must not overlap rows (x %lld, cache b %lld, t %lld for C=%d, T=%d)",
                (long long)x_stride_b, (long long)cache_stride_b, (long long)cache_stride_t, C, T);
  const int64_t n = (int64_t)B * C;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), B, C, T, x, x_stride_b, cache, cache_stride_b,
                     cache_stride_t, lengths);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_greedy_pick_f32(int rows, int cols, const float* x, int64_t ld, int64_t* cur, int64_t* ids,
                                   int Tmax, float* margins, int t_base, int n_margins, int* lengths,
                                   int64_t* pos, void* stream) {
  MTX_CHECK_SHAPE(rows >= 1 && cols >= 1 && Tmax >= 1, "rows, cols, Tmax must be >= 1 (got %d, %d, %d)", rows,
                  cols, Tmax);
  MTX_CHECK_ARG(x && cur && ids && lengths, "x, cur, ids, lengths: null pointer");
  MTX_CHECK_ARG(ld >= cols, "ld=%lld < cols=%d", (long long)ld, cols);
  MTX_CHECK_ARG(margins == nullptr || n_margins >= 1, "n_margins must be >= 1 with a margin buffer");
  hipLaunchKernelGGL(greedy_pick_kernel, dim3((rows + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream),
                     rows, cols, x, ld, cur, ids, Tmax, margins, t_base, n_margins, lengths, pos);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_head_pick_f32(int rows, int K, int V, const float* x, int64_t ldx, const float* pws, int pks,
                                 const float* pbias, const float* ln_gamma, const float* ln_beta, float eps,
                                 const float* W, int64_t ldw, const float* bias, int64_t* cur, int64_t* ids, int Tmax,
                                 float* margins, int t_base, int n_margins, int* lengths, int64_t* pos,
                                 void* stream) {
  MTX_CHECK_SHAPE(rows >= 1 && K >= 1 && V >= 1 && Tmax >= 1, "rows, K, V, Tmax must be >= 1");
  MTX_CHECK_SHAPE(V <= 64 * 4 && K <= 8192, "head_pick: needs V <= 256 and K <= 8192 (got V=%d, K=%d)", V, K);
  MTX_CHECK_ARG(x && W && cur && ids && lengths, "x, W, cur, ids, lengths: null pointer");
  MTX_CHECK_ARG(ldx >= K && ldw >= V, "head_pick: bad row strides");
  MTX_CHECK_ARG(margins == nullptr || n_margins >= 1, "n_margins must be >= 1 with a margin buffer");
  MTX_CHECK_ARG(ln_gamma ? ln_beta != nullptr : pws == nullptr,
                "head_pick: pending partials need the LayerNorm (gamma and beta)");
  MTX_CHECK_SHAPE(!ln_gamma || K <= 1024, "head_pick: the LayerNorm input mode needs K <= 1024 (got %d)", K);
  MTX_CHECK_ARG(!pws || (pks >= 1 && pks <= 8), "head_pick: 1 to 8 pending partial products");
  MTX_CHECK_ARG(std::isfinite(eps) && eps >= 0.f, "head_pick: eps must be finite and >= 0");
  const PendingLn pl{pws, pks, pbias, nullptr, 0, ln_gamma, ln_beta, eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpl = (V + 63) / 64;
  const int vp = vpl <= 1 ? 1 : (vpl <= 2 ? 2 : 4);
  const size_t lds = ((size_t)((K + 3) & ~3) + (size_t)kHpW * 64 * vp) * sizeof(float);
#define HP(VP) hipLaunchKernelGGL(head_pick_kernel<VP>, dim3(rows), dim3(64 * kHpW), lds, st, rows, K, V, x, ldx, pl, W, ldw, bias, cur, ids, Tmax, margins, t_base, n_margins, lengths, pos)
  if (vpl <= 1) HP(1);
  else if (vpl <= 2) HP(2);
  else HP(4);
#undef HP
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_embedding2_ln_fwd_f32(const float* wa, int64_t lda, int64_t Va, const int64_t* ia,
                                         const float* wb, int64_t ldb, int64_t Vb, const int64_t* ib,
                                         int64_t ib_stride, float* out, int64_t ldo, int64_t n, int C,
                                         const float* gamma, const float* beta, float eps, float* y, int64_t ldy,
                                         void* stream) {
  MTX_CHECK_ARG(wa && ia && wb && ib && out && gamma && beta && y, "embedding2_ln: null pointer");
  MTX_CHECK_SHAPE(n >= 0 && C >= 1 && C <= 64 * 32 && Va >= 1 && Vb >= 1 && lda >= C && ldb >= C && ldo >= C &&
                      ldy >= C && ib_stride >= 0,
                  "embedding2_ln: bad shape (C must be in [1, 2048])");
  if (n == 0) return MTX_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpl = (C + 63) / 64;
#define E2L(VP) hipLaunchKernelGGL(embed2_ln_kernel<VP>, dim3((unsigned)n), dim3(64), 0, st, wa, lda, Va, ia, wb, ldb, Vb, ib, ib_stride, out, ldo, C, gamma, beta, eps, y, ldy)
  if (vpl <= 1) E2L(1);
  else if (vpl <= 2) E2L(2);
  else if (vpl <= 4) E2L(4);
  else if (vpl <= 6) E2L(6);
  else if (vpl <= 8) E2L(8);
  else if (vpl <= 12) E2L(12);
  else if (vpl <= 16) E2L(16);
  else E2L(32);
#undef E2L
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_embedding2_fwd_f32(const float* wa, int64_t lda, int64_t Va, const int64_t* ia, const float* wb,
                                      int64_t ldb, int64_t Vb, const int64_t* ib, int64_t ib_stride, float* out,
                                      int64_t ldo, int64_t n, int C, void* stream) {
  MTX_CHECK_ARG(wa && ia && wb && ib && out, "embedding2: null pointer");
  MTX_CHECK_SHAPE(n >= 0 && C >= 1 && Va >= 1 && Vb >= 1 && lda >= C && ldb >= C && ldo >= C && ib_stride >= 0,
                  "embedding2: bad shape");
  if (n == 0) return MTX_OK;
  const int blocks = (int)std::min<int64_t>((n * C + 255) / 256, 16384);
  hipLaunchKernelGGL(embed2_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), wa, lda, Va, ia,
                     wb, ldb, Vb, ib, ib_stride, out, ldo, n, C);
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_decode_advance(int B, int* lengths, int64_t* pos, void* stream) {
  MTX_CHECK_SHAPE(B >= 1, "B must be >= 1 (got %d)", B);
  MTX_CHECK_ARG(lengths != nullptr, "lengths: null pointer");
  hipLaunchKernelGGL(advance_kernel, dim3((B + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), B,
                     lengths, pos);
  MTX_LAUNCHED();
  return MTX_OK;
}
