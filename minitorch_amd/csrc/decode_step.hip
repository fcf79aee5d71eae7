// Greedy decode steps of a GPT in one persistent, cooperative launch, for
// gfx950 (MI355X).
//
// mtx_decode_step_f32 replaces one iteration of the reference's generation
// loop (GPT.generate, transformer.py:93-104: the forward of
// transformer.py:80-91 for the newest position, then the greedy pick) when
// the keys and values of earlier positions sit in a cache.  The multi-launch
// decode step (decode.hip and gemm.hip's step kernels) needs 2 + 5 launches
// per block, each costing a few microseconds of launch and drain however
// small its work; here the step is one launch whose workgroups all stay
// resident (hipLaunchCooperativeKernel fails rather than start a grid that
// does not fit) and meet at grid-wide barriers between stages.  One launch
// can also run several consecutive token steps, with one more barrier after
// each step's pick:
//
//   stage A, per block, items (pair of sequences, head): the block's input
//     rows (embeddings for the first block, else the previous block's
//     residual plus its pending fc2 partial products and bias), ln1, the
//     head's q/k/v columns with the cache writes, the decode attention over
//     the cached keys, and the head's share of out_proj (its 64 rows of the
//     weight) as a partial product per head;
//   barrier;
//   stage B, per block, items (8 rows, 48 hidden columns at C = 384, else
//     64): the residual plus
//     the head partials of out_proj and its bias (written back as the
//     residual by the first column slab), ln2, fc1 + GELU on the slab (its
//     weight columns staged in LDS by direct loads while stage A runs), and
//     fc2's partial product over the slab's 64 rows of its weight;
//   barrier;
//   after the last block, items (row): the residual plus the last fc2
//     partials and bias, ln_f, lm_head and the pick with its bookkeeping.
//
// The barrier is a set of 64-bit arrival counters in device memory (the
// workspace), added to by one thread per workgroup and polled by one wave
// with agent-scope atomics; each launch counts from the base the launch
// before it left.  Every
// wait is bounded by the 100 MHz wall clock: a wait that runs out sets the
// workspace's error word and the workgroup leaves the kernel; waiting
// workgroups see the word and leave too, and a later launch on the same
// workspace returns at its start.  Sums run in fixed orders, so the step is
// deterministic.
#include "mtx_common.h"
#include "decode_pick.h"

#include <algorithm>
#include <cmath>
#include <mutex>

namespace mtx {
namespace {

constexpr int kPsW = 16;         // waves per workgroup
constexpr int kPsT = 64 * kPsW;  // threads per workgroup
constexpr int kPsD = 64;         // head size
constexpr int kPsMaxC = 512;
constexpr int kPsMaxH = kPsMaxC / kPsD;
constexpr int kPsS = 2;          // sequences per stage-A item
constexpr int kPsR = 8;          // rows per stage-B item
constexpr int kPsHS = 64;        // most hidden columns per stage-B item
constexpr int kPsMaxT = 1024;    // cache rows (scores of kPsS rows in LDS)
constexpr int kPsMaxL = 16;
constexpr int kPsMaxV = 256;
// barrier words (unsigned), each on its own 128-byte line: kBarNC arrival
// counters (64-bit; workgroup i adds to counter i mod kBarNC, and wave 0 of a
// waiting workgroup reads kBarNC / 64 per lane), the launch base (64-bit),
// the error word
#ifndef MTX_DS_BAR_COUNTERS
#define MTX_DS_BAR_COUNTERS 128
#endif
constexpr int kBarNC = MTX_DS_BAR_COUNTERS;
constexpr int kBarPL = kBarNC / 64;  // counters per polling lane
static_assert(kBarNC % 64 == 0 && (kBarNC & (kBarNC - 1)) == 0, "whole counters per lane of wave 0");
// hidden columns per stage-B item: 48 at C = 384 (the MLP width 1536 in 32
// slabs: with 64 sequences, 8 row groups x 32 slabs = 256 items, one per CU,
// where 64-column slabs leave 64 CUs idle in stage B), else 64
template <int C>
constexpr int ps_hs() { return C == 384 ? 48 : kPsHS; }
inline int ps_hs_host(int C) { return C == 384 ? 48 : kPsHS; }
constexpr int kBarCount = 0, kBarBase = 32 * kBarNC, kBarErr = kBarBase + 32, kBarBytes = 4 * (kBarErr + 32);

struct PsArgs {
  int NL, B, C, H, F, V, Tmax;
  float scale;
  const float* tok;
  int64_t ntok;
  const float* posw;
  int64_t npos;
  const float* lnfg;
  const float* lnfb;
  float epsf;
  const float* wh;
  const float* bh;
  int64_t* cur;
  int64_t* ids;
  float* margins;
  int t_base, nm;
  int* lengths;
  int64_t* pos;
  float* X0;  // residual after a block's attention half ... (B, C)
  float* X1;  // ... and the block input (B, C)
  float* P1;  // out_proj partial products per head (H, B, C)
  float* P2;  // fc2 partial products per column slab (F / 64, B, C)
  unsigned* bar;
  int64_t limit;  // wall-clock ticks a barrier wait may take; < 0: fail at once
  int steps;      // token steps in this launch
  mtx_decode_layer L[kPsMaxL];
};
static_assert(sizeof(PsArgs) <= 4096, "kernel arguments are limited to 4 KiB");

constexpr int kPsOpart = 8192;  // out_proj group partial sums, floats
struct PsStageA {
  float xs[kPsS][kPsMaxC];
  union {
    float buf[kPsW * kPsS * 3 * kPsD];  // wave partial sums, then key-group partial outputs
    float opart[kPsOpart];              // then out_proj group partial sums
  };
  float qkv[kPsS][3 * kPsD];
  float o[kPsS][kPsD];
  float red[kPsW];
  float sc[kPsS][kPsMaxT];
};
struct PsStageB {
  float xs[kPsR][kPsMaxC + 4];  // (rows 16 bytes apart in the banks)
  float hs[kPsR][kPsHS];
};
struct PsHead {
  float xs[kPsMaxC];
  float part[kPsW * 64 * 4];
};
union PsSmem {
  PsStageA a;
  PsStageB b;
  PsHead h;
};
// Stage B's slab region: fc1's weights [C][HS] (filled by direct loads),
// then the fc1 partial sums [kPsW][kPsR][HS], then the fc2 half sums
// [2][kPsR][C].  Where it fits beside the union (C <= 384) it has LDS of its
// own and a workgroup requests its first stage-B slab at the start of stage
// A; otherwise it lies over stage A's data, after stage B's rows, and the
// request waits for the end of stage A.
template <int C>
struct PsLds {
  static constexpr int kUnion = (int)(sizeof(PsSmem) / sizeof(float));
  static constexpr int kSlab = C * ps_hs<C>();
  static constexpr bool kApart = (kUnion + kSlab) * (int)sizeof(float) <= 160 * 1024 - 256;
  static constexpr int kSlabOff = kApart ? kUnion : (int)(sizeof(PsStageB) / sizeof(float));
  static constexpr int kTotal = kApart ? kUnion + kSlab : (kSlabOff + kSlab > kUnion ? kSlabOff + kSlab : kUnion);
  static_assert(kPsW * kPsR * ps_hs<C>() <= kSlab && 2 * kPsR * C <= kSlab, "partial sums fit the slab region");
  static_assert(kSlabOff % 4 == 0, "16-byte aligned slab");
};

// Data that crosses workgroups within a launch (the residual rows X0/X1, the
// partial products P1/P2, and between token steps the next input ids, the
// lengths and the position) is written and read with device-scope
// accesses (relaxed atomics at agent scope: sc1 loads and stores, coherent
// across the XCDs' L2 caches).  Everything else a stage reads -- weights,
// the caches, the step's inputs -- is written before the launch or by the
// same workgroup, and stays in the L2 caches across the barriers.
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_dev_i(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_dev_i(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A load at a 32-bit byte offset from a wave-uniform base: the form the
// compiler turns into one scalar base register pair plus one vector offset
// register, instead of a 64-bit address per load.
template <typename T>
__device__ __forceinline__ T ld_off(const float* base, unsigned byte_off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}

// A LayerNorm's gamma and beta at the lane's columns lane + 64 i, requested
// at the start of an item so that they are in registers when the row is
struct LnPar {
  float g[kPsMaxC / 64], b[kPsMaxC / 64];
};
template <int C>
__device__ __forceinline__ void ln_load(LnPar& p, const float* __restrict__ g, const float* __restrict__ be,
                                        int lane) {
#pragma unroll
  for (int i = 0; i < C / 64; ++i) {
    p.g[i] = ld_off<float>(g, 4u * (unsigned)(lane + 64 * i));
    p.b[i] = ld_off<float>(be, 4u * (unsigned)(lane + 64 * i));
  }
}

// LayerNorm of one LDS row of C <= 512 values by one wave, in place (the
// arithmetic of layernorm_fwd_kernel)
template <int C>
__device__ __forceinline__ void ps_ln_row(float* __restrict__ row, int lane, const LnPar& p, float eps) {
  float v[kPsMaxC / 64];
#pragma unroll
  for (int i = 0; i < kPsMaxC / 64; ++i) {
    const int n = lane + 64 * i;
    v[i] = n < C ? row[n] : 0.f;
  }
  float mean, sd;
  ln_stats<kPsMaxC / 64>(v, lane, C, eps, mean, sd);
#pragma unroll
  for (int i = 0; i < C / 64; ++i) row[lane + 64 * i] = ln_apply(v[i], sd, p.g[i], p.b[i]);
}

// Element n of row b entering a block after the first: the residual X0[b]
// plus the previous block's fc2 partial products (summed in slab order) and
// its bias -- (sum + bias) + residual, the grouping of the chain's reduce
template <int C>
__device__ __forceinline__ float ps_pending(const PsArgs& a, const float* __restrict__ bias, int b, int n) {
  constexpr int ns = 4 * C / ps_hs<C>();   // slabs of the MLP width F = 4C
  constexpr int NB = ns <= 24 ? ns : 16;   // loads in flight
  const int64_t stride = (int64_t)a.B * C;
  const unsigned off = (unsigned)(b * C + n);
  float s = 0.f;
#pragma unroll
  for (int s0 = 0; s0 < ns; s0 += NB) {
    float pv[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) pv[q] = ld_dev(a.P2 + (int64_t)(s0 + q) * stride + off);
#pragma unroll
    for (int q = 0; q < NB; ++q) s += pv[q];
  }
  float t = s + bias[n];
  t += ld_dev(a.X0 + off);
  return t;
}

// Grid-wide barrier over arrival counters that only grow, spread over kBarNC
// counters on separate lines (with one counter for the whole grid, the
// arrivals and polls on its one line queued behind each other and each
// barrier took about 1 us longer; with 64 counters for 256 workgroups a
// token step took 2 us longer than with 128).  A launch reads the counters' total at its
// start from the base word (written by the launch before it, so launches of
// different grid sizes may share a workspace); its k-th barrier (k = 1, 2,
// ...) is complete when the total reaches base + k G, and its workgroup 0
// leaves the final total as the next launch's base.  `next` (lanes of wave
// 0) is this workgroup's next target.  Each thread first waits for its own
// stores (the device-scope stores are acknowledged once they are visible
// across the device), the workgroup barrier then covers every thread, thread
// 0 adds to its counter, and wave 0 polls: lane i reads counters i, i + 64,
// ... and the lanes sum them (each counter only grows, so a total that reaches the
// target means every arrival happened).  No cache write-back or invalidation
// is needed, so the L2 caches keep the weights across stages.
// Arrival and wait are separate so that loads that do not depend on the
// stage before (the next stage's first weights) can be issued between them:
// issued before the arrival, the arrival's wait for this thread's stores
// would wait for them too (one counter covers loads and stores).
// ps_wait returns false when the step must end: this wait ran out, or
// another workgroup's did.
__device__ __forceinline__ void ps_arrive(const PsArgs& a) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(reinterpret_cast<unsigned long long*>(a.bar + kBarCount + 32 * (blockIdx.x % kBarNC)),
                           1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool ps_wait(const PsArgs& a, int* flag, unsigned long long& next) {
  const unsigned long long target = next;
  next += gridDim.x;
  if (threadIdx.x < 64) {
    unsigned* err = a.bar + kBarErr;
    int ok = 1;
    const int64_t t0 = wall_clock64();
    while (true) {
      // (a negative limit fails before the first poll, so that the failure
      // does not depend on how far the other workgroups have come)
      if (a.limit >= 0) {
        unsigned long long s = 0;
#pragma unroll
        for (int c = 0; c < kBarPL; ++c)
          s += __hip_atomic_load(reinterpret_cast<unsigned long long*>(a.bar + kBarCount + 32 * (threadIdx.x + 64 * c)),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int o = 1; o < 64; o *= 2) s += __shfl_xor(s, o, 64);
        if (s >= target) break;
      }
      if (a.limit < 0 || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u ||
          wall_clock64() - t0 > a.limit) {
        if (threadIdx.x == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) *flag = ok;
  }
  __syncthreads();
  if (*flag != 0) return true;
  __builtin_amdgcn_s_waitcnt(0);  // no load issued between arrival and wait outlives the workgroup
  return false;
}

__device__ __forceinline__ bool ps_barrier(const PsArgs& a, int* flag, unsigned long long& next) {
  ps_arrive(a);
  return ps_wait(a, flag, next);
}

// ---- stage A: (pair of sequences, head) ----
// Weights of an item do not depend on the previous stage: a workgroup's
// first stage-A item has its first weight batch requested between the
// arrival and the wait of the barrier that opens the stage (PreA), so that
// latency overlaps the wait.  (Stage B's weights requested into registers
// that way pushed the kernel past 128 VGPRs into spills; its fc1 slab goes
// to LDS by direct loads instead, requested at the start of stage A, and
// fc2's weights are requested around fc1.)
constexpr int kPsNPL = 3 * kPsD / 64;   // q, k, v columns of the head per lane
constexpr int kPsBA = 36 / kPsNPL;      // weight rows per load batch in stage A
struct PreA {
  float wv[kPsBA][kPsNPL];
};

// the thread index, opaque to the compiler, so that values derived from it
// are computed per item instead of being hoisted out of the kernel's layer
// and item loops (which would keep them all live)
__device__ __forceinline__ int ps_tid() {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  return tid;
}

// stage A's weight rows [kb, kb + kPsBA) of wave w's range, the head's q, k
// and v columns (rows clamped to the matrix)
template <int C>
__device__ __forceinline__ void attn_load(const mtx_decode_layer& Ly, int h, int lane, int kb, PreA& p) {
  constexpr int D = kPsD;
  const int64_t ldw = 3 * (int64_t)C;
  unsigned col[kPsNPL];  // byte offsets of the lane's columns
#pragma unroll
  for (int t = 0; t < kPsNPL; ++t) {
    const int jj = lane + 64 * t;
    col[t] = 4u * (unsigned)((jj / D) * C + h * D + jj % D);
  }
#pragma unroll
  for (int j = 0; j < kPsBA; ++j) {
    const float* __restrict__ wr = Ly.w_qkv + (int64_t)min(kb + j, C - 1) * ldw;
#pragma unroll
    for (int t = 0; t < kPsNPL; ++t) p.wv[j][t] = ld_off<float>(wr, col[t]);
  }
}

template <int C>
__device__ __forceinline__ void attn_prefetch(const PsArgs& a, int l, int item, PreA& p) {
  const int tid = ps_tid();
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  attn_load<C>(a.L[l], item % a.H, lane, w * (C / kPsW), p);
}

template <int C>
__device__ __forceinline__ void ps_attn_item(const PsArgs& a, int l, int item, PsStageA& sm, PreA& pre,
                                             bool prefetched) {
  constexpr int D = kPsD, S = kPsS;
  constexpr int NC = 3 * D;     // the head's q, k and v columns
  constexpr int NPL = kPsNPL;   // of which each lane owns NPL
  constexpr int WS = kPsW / S;  // waves per sequence in the attention
  constexpr int TPS = 64 * WS;
  constexpr int DV = D / 4, NGS = TPS / DV;  // value slices, key groups per sequence
  constexpr int kB = kPsBA;
  static_assert(S * NGS * D <= kPsW * S * NC, "key-group partials fit the wave-sum buffer");
  const mtx_decode_layer& Ly = a.L[l];
  const int B = a.B, H = a.H;
  const int b0 = (item / H) * S, h = item % H;
  const int tid = ps_tid();
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // q, k, v: wave w sums over weight rows [k0, k1) in batches of kB rows
  // whose loads are all issued before their products; the first batch is
  // requested before the input rows are read (or before the stage's barrier)
  const int kcnt = C / kPsW;
  const int k0 = w * kcnt, k1 = k0 + kcnt;
  if (!prefetched) attn_load<C>(Ly, h, lane, k0, pre);
  LnPar lp;
  if (w < S) ln_load<C>(lp, Ly.ln1_gamma, Ly.ln1_beta, lane);

  __syncthreads();  // the previous item's LDS reads are done
  {
    int64_t ra[S];
    int64_t rb = 0;
    if (l == 0) {
      rb = ld_dev_i(a.pos);
      rb = rb < 0 ? 0 : (rb >= a.npos ? a.npos - 1 : rb);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        int64_t r = b0 + s < B ? ld_dev_i(a.cur + b0 + s) : 0;
        ra[s] = r < 0 ? 0 : (r >= a.ntok ? a.ntok - 1 : r);
      }
    }
    for (int i = tid; i < S * C; i += kPsT) {
      const int s = i / C, n = i % C, b = b0 + s;
      float t = 0.f;
      if (b < B) {
        if (l == 0) t = a.tok[(s == 0 ? ra[0] : ra[S - 1]) * C + n] + a.posw[rb * C + n];
        else t = ps_pending<C>(a, a.L[l - 1].b_fc2, b, n);
        if (h == 0) st_dev(a.X1 + (int64_t)b * C + n, t);
      }
      sm.xs[s][n] = t;
    }
  }
  __syncthreads();
  if (w < S) ps_ln_row<C>(sm.xs[w], lane, lp, Ly.ln1_eps);
  __syncthreads();

  float acc[S][NPL];
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < NPL; ++t) acc[s][t] = 0.f;
  for (int kb = k0; kb < k1; kb += kB) {
    if (kb != k0) attn_load<C>(Ly, h, lane, kb, pre);
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (kb + j < k1) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const float xv = sm.xs[s][kb + j];
#pragma unroll
          for (int t = 0; t < NPL; ++t) acc[s][t] = fmaf(xv, pre.wv[j][t], acc[s][t]);
        }
      }
    }
  }
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int t = 0; t < NPL; ++t) sm.buf[(w * S + s) * NC + lane + 64 * t] = acc[s][t];

  __syncthreads();
  for (int i = tid; i < S * NC; i += kPsT) {
    const int s = i / NC, jj = i % NC;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kPsW; ++q) v += sm.buf[(q * S + s) * NC + jj];
    const int pt = jj / D, e = jj % D;
    v += Ly.b_qkv[pt * C + h * D + e];
    sm.qkv[s][jj] = v;
    const int b = b0 + s;
    if (pt > 0 && b < B) {
      const int t = ld_dev_i(a.lengths + b) - 1;
      if (t >= 0 && t < a.Tmax)
        (pt == 1 ? Ly.k_cache : Ly.v_cache)[((int64_t)b * a.Tmax + t) * C + h * D + e] = v;
    }
  }
  __syncthreads();

  // ---- attention: waves [sg*WS, sg*WS + WS) take sequence b0 + sg ----
  {
    const int sg = w / WS, lt = tid % TPS;
    const int b = b0 + sg;
    const int len = b < B ? ld_dev_i(a.lengths + b) : 0;
    const int L = min(max(len, 0), a.Tmax);
    const int newrow = (len >= 1 && len <= a.Tmax) ? len - 1 : -1;  // the row this step wrote
    const int64_t cst = C, csb = (int64_t)a.Tmax * C;
    float* __restrict__ scs = sm.sc[sg];
    const float* __restrict__ qv = sm.qkv[sg];
    // scores (log2 units): four threads per key, a quarter of D each; a
    // thread's keys two at a time, both rows requested together (one memory
    // round trip for up to 2 TPS / 4 keys)
    const float c = a.scale * kLog2e;
    constexpr int DQ = D / 4, KP = TPS / 4;
    const int kq = lt >> 2, qd = lt & 3;
    float qr[DQ];
#pragma unroll
    for (int e = 0; e < DQ; ++e) qr[e] = qv[qd * DQ + e] * c;
    const float* __restrict__ kb0 = Ly.k_cache + (int64_t)min(b, B - 1) * csb + h * D + qd * DQ;
    float mx = -INFINITY;
    for (int j0 = kq; j0 < L; j0 += 2 * KP) {
      float kr[2][DQ];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = min(j0 + u * KP, L - 1);  // a row past L is not used
#pragma unroll
        for (int e = 0; e < DQ; e += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(kb0 + (int64_t)j * cst + e);
          kr[u][e] = v[0]; kr[u][e + 1] = v[1]; kr[u][e + 2] = v[2]; kr[u][e + 3] = v[3];
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int j = j0 + u * KP;
        if (j == newrow) {
#pragma unroll
          for (int e = 0; e < DQ; ++e) kr[u][e] = qv[D + qd * DQ + e];
        }
        float sv = 0.f;
#pragma unroll
        for (int e = 0; e < DQ; ++e) sv = fmaf(qr[e], kr[u][e], sv);
        sv += __shfl_xor(sv, 1, 64);
        sv += __shfl_xor(sv, 2, 64);
        if (j < L) {
          if (qd == 0) scs[j] = sv;
          mx = fmaxf(mx, sv);
        }
      }
    }

    // the value rows of the first 8 key groups, requested before the
    // softmax so that their latency overlaps it (rows past L are not used;
    // the row this step wrote is taken from LDS)
    const int dv = lt % DV, kg = lt / DV;
    const float* __restrict__ vb0 = Ly.v_cache + (int64_t)min(b, B - 1) * csb + h * D + 4 * dv;
    constexpr int VPF = 8;
    f32x4 vpre[VPF];
    if (L > 0) {
#pragma unroll
      for (int i = 0; i < VPF; ++i)
        vpre[i] = *reinterpret_cast<const f32x4*>(vb0 + (int64_t)min(kg + i * NGS, L - 1) * cst);
    }
    mx = wave_max(mx);
    if (lane == 0) sm.red[w] = mx;
    __syncthreads();
    mx = sm.red[sg * WS];
#pragma unroll
    for (int q = 1; q < WS; ++q) mx = fmaxf(mx, sm.red[sg * WS + q]);
    __syncthreads();
    float sum = 0.f;
    for (int j = lt; j < L; j += TPS) {
      const float p = __builtin_amdgcn_exp2f(scs[j] - mx);
      scs[j] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) sm.red[w] = sum;
    __syncthreads();  // also publishes every p_j
    float lsum = 0.f;
#pragma unroll
    for (int q = 0; q < WS; ++q) lsum += sm.red[sg * WS + q];

    // o[d] = sum_j p_j v[j][d] / l
    f32x4 av = zero4();
#pragma unroll
    for (int i = 0; i < VPF; ++i) {
      const int j = kg + i * NGS;
      if (j < L) av += scs[j] * (j == newrow ? *reinterpret_cast<const f32x4*>(qv + 2 * D + 4 * dv) : vpre[i]);
    }
#pragma unroll 4
    for (int j = kg + VPF * NGS; j < L; j += NGS) {
      const f32x4 vv = j == newrow ? *reinterpret_cast<const f32x4*>(qv + 2 * D + 4 * dv)
                                   : *reinterpret_cast<const f32x4*>(vb0 + (int64_t)j * cst);
      av += scs[j] * vv;
    }
    *reinterpret_cast<f32x4*>(sm.buf + (sg * NGS + kg) * D + 4 * dv) = av;
    __syncthreads();
    if (lt < D) {
      float r = 0.f;
#pragma unroll 8
      for (int g = 0; g < NGS; ++g) r += sm.buf[(sg * NGS + g) * D + lt];
      sm.o[sg][lt] = L > 0 ? r / lsum : 0.f;
    }
  }
  __syncthreads();

  // this head's rows of out_proj: thread (eg, cg) takes rows
  // [64h + RPE eg, + RPE) of columns [4cg, 4cg + 4)
  constexpr int CG = C / 4;
  constexpr int EG = (kPsT / CG) >= 16 ? 16 : 8;
  constexpr int RPE = D / EG;
  static_assert(CG * EG <= kPsT && EG * S * C <= kPsOpart, "out_proj thread split");
  const bool op_thread = tid < CG * EG;
  const int cg = tid % CG, eg = tid / CG;
  f32x4 wo4[RPE];
  if (op_thread) {
#pragma unroll
    for (int r = 0; r < RPE; ++r)
      wo4[r] = ld_off<f32x4>(Ly.w_out + (int64_t)(h * D) * C, 4u * (unsigned)((eg * RPE + r) * C + 4 * cg));
  }
  // ---- this head's share of out_proj: o_h (S x 64) times weight rows
  // [64h, 64h + 64): each row group's sum (rows ascending, one fused
  // multiply-add per term), then the EG group sums in order ----
  if (op_thread) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      f32x4 po = zero4();
#pragma unroll
      for (int r = 0; r < RPE; ++r) {
        const float ov = sm.o[s][eg * RPE + r];
#pragma unroll
        for (int c = 0; c < 4; ++c) po[c] = fmaf(ov, wo4[r][c], po[c]);
      }
      *reinterpret_cast<f32x4*>(sm.opart + (eg * S + s) * C + 4 * cg) = po;
    }
  }
  __syncthreads();
  for (int i = tid; i < S * C; i += kPsT) {
    const int s = i / C, n = i % C;
    if (b0 + s < B) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < EG; ++g) v += sm.opart[(g * S + s) * C + n];
      st_dev(a.P1 + ((int64_t)h * B + b0 + s) * C + n, v);
    }
  }
}

// ---- stage B: (8 rows, HS = 48 or 64 hidden columns) ----
// fc1: wave w sums weight rows [w kc, w kc + kc) for the slab's columns, the
// slab staged in LDS; fc2: thread (half, n), n < C, sums the slab's hidden
// columns [HS/2 half, HS/2 half + HS/2) for all 8 rows of column n, and the
// two halves are added through LDS
// fc2 weight rows (24 of a thread's 32 with 64-column slabs, 18 of 24 with
// 48) requested before fc1; the rest after it (all 32 before fc1 measured
// slower, 0.1945 against 0.1937 ms per step)
template <int C>
constexpr int ps_w2e() { return ps_hs<C>() == 64 ? 24 : 18; }
template <int C>
struct PreB {
  float w2v[ps_hs<C>() / 2];
};

typedef __attribute__((address_space(3))) void lds_void;

// fc1's weight slab of an item (rows 0 .. C-1, columns j0 .. j0+63) into
// w1s[k][64] by direct buffer loads into LDS: no registers, so a workgroup's
// first item has it requested before the stage (at the start of stage A, or
// between the arrival and the wait of the barrier before the stage where the
// slab lies over stage A's LDS).  One wave load moves four rows (1 KiB);
// completion is the wave's vmcnt.
template <int C>
__device__ __forceinline__ void mlp_dma(const mtx_decode_layer& Ly, int F, int item, float* w1s) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int HS = ps_hs<C>();
  constexpr int RB = HS * (int)sizeof(float);  // bytes per slab row
  constexpr int NI = C * RB / 1024;            // wave loads of 1 KiB
  constexpr int PW = (NI + kPsW - 1) / kPsW;
  static_assert(C * RB % 1024 == 0 && RB % 16 == 0, "whole wave loads, 16-byte pieces within a row");
  const int j0 = (item % (F / HS)) * HS;
  const int tid = ps_tid();
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bytes = ((C - 1) * F + HS) * (int)sizeof(float);
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Ly.w_fc1 + j0), (short)0, bytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int ins = w + i * kPsW;  // (wave-uniform)
    if (NI % kPsW == 0 || ins < NI) {
      // the slab's bytes [1024 ins, 1024 ins + 1024), 16 per lane: row k,
      // byte cb of the row
      const int b = 1024 * ins + 16 * lane;
      const int k = b / RB, cb = b % RB;
      const uint32_t voff = (uint32_t)(k * F * (int)sizeof(float) + cb);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(w1s + ins * 256), 16, voff, 0, 0, 0);
    }
  }
#endif
}

// fc2's weights of the thread's rows [J0, J1) of its half
template <int C, int J0, int J1>
__device__ __forceinline__ void mlp_load2(const mtx_decode_layer& Ly, int F, int item, PreB<C>& p) {
  constexpr int HS = ps_hs<C>();
  const int j0 = (item % (F / HS)) * HS;
  const int tid = ps_tid();
  if (tid < 2 * C) {
    const float* __restrict__ wr = Ly.w_fc2 + (int64_t)(j0 + (HS / 2) * (tid / C) + J0) * C;
    const unsigned n2 = 4u * (unsigned)(tid % C);
#pragma unroll
    for (int j = J0; j < J1; ++j, wr += C) p.w2v[j] = ld_off<float>(wr, n2);
  }
}

template <int C>
__device__ __forceinline__ void ps_mlp_item(const PsArgs& a, int l, int item, PsStageB& sm, float* big, bool prefetched) {
  const mtx_decode_layer& Ly = a.L[l];
  constexpr int HS = ps_hs<C>();
  const int B = a.B, F = a.F;
  const int ns = F / HS;
  const int rg = item / ns, sl = item % ns;
  const int m0 = rg * kPsR, j0 = sl * HS;
  const int tid = ps_tid();
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int kc = C / kPsW;
  const int k0 = w * kc;
  PreB<C> pre;
  if (!prefetched) {
    __syncthreads();  // the previous item's LDS reads are done
    mlp_dma<C>(Ly, F, item, big);
  }
  LnPar lp;
  if (w < kPsR) ln_load<C>(lp, Ly.ln2_gamma, Ly.ln2_beta, lane);

  __syncthreads();  // the previous item's LDS reads are done
  const int64_t hstride = (int64_t)B * C;
  for (int i = tid; i < kPsR * C; i += kPsT) {
    const int m = i / C, n = i % C, b = m0 + m;
    float t = 0.f;
    if (b < B) {
      const unsigned off = (unsigned)(b * C + n);
      constexpr int NH = C / kPsD;  // heads (H = C / 64, checked on the host)
      float pv[NH];
#pragma unroll
      for (int q = 0; q < NH; ++q) pv[q] = ld_dev(a.P1 + (int64_t)q * hstride + off);
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < NH; ++q) s += pv[q];
      t = s + Ly.b_out[n];
      t += ld_dev(a.X1 + off);
      if (sl == 0) st_dev(a.X0 + off, t);
    }
    sm.xs[m][n] = t;
  }
  __syncthreads();
  if (w < kPsR) ps_ln_row<C>(sm.xs[w], lane, lp, Ly.ln2_eps);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's slab rows have landed
  __syncthreads();
  // the first of fc2's weight rows, requested before fc1
  mlp_load2<C, 0, ps_w2e<C>()>(Ly, F, item, pre);

  const float* __restrict__ w1s = big;
  float* __restrict__ part = big;  // [kPsW][kPsR][HS], over the consumed slab
  static_assert(kc % 4 == 0, "whole groups of four weight rows");
  if constexpr (HS == kPsHS) {
    // lane = hidden column, all 8 rows; four weight rows at a time, the row
    // values as one 16-byte broadcast read per row (terms added in
    // ascending k)
    float acc[kPsR];
#pragma unroll
    for (int m = 0; m < kPsR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int i = 0; i < kc; i += 4) {
      float wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) wv[u] = w1s[(k0 + i + u) * HS + lane];
#pragma unroll
      for (int m = 0; m < kPsR; ++m) {
        const f32x4 x4 = *reinterpret_cast<const f32x4*>(&sm.xs[m][k0 + i]);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[m] = fmaf(x4[u], wv[u], acc[m]);
      }
      // keep the scheduler from hoisting every row value's LDS read at once
      if (i % 8 == 4) __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // every wave's slab reads are done
#pragma unroll
    for (int m = 0; m < kPsR; ++m) part[(w * kPsR + m) * HS + lane] = acc[m];
  } else {
    // 48 columns: lane (cg, rp) takes columns cg, cg + 16, cg + 32 of rows
    // 2 rp and 2 rp + 1, so that every lane works; per output the terms are
    // still added in ascending k
    static_assert(HS == 48 && kPsR == 8, "48 columns = 3 x 16 lanes, 8 rows = 4 x 2");
    const int cg = lane & 15, rp = lane >> 4;
    float acc[2][3];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[r][c] = 0.f;
#pragma unroll
    for (int i = 0; i < kc; i += 4) {
      float wv[4][3];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int c = 0; c < 3; ++c) wv[u][c] = w1s[(k0 + i + u) * HS + cg + 16 * c];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const f32x4 x4 = *reinterpret_cast<const f32x4*>(&sm.xs[2 * rp + r][k0 + i]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int c = 0; c < 3; ++c) acc[r][c] = fmaf(x4[u], wv[u][c], acc[r][c]);
      }
      if (i % 8 == 4) __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();  // every wave's slab reads are done
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < 3; ++c) part[(w * kPsR + 2 * rp + r) * HS + cg + 16 * c] = acc[r][c];
  }

  // the rest of fc2's weights, requested before the fc1 reduce
  mlp_load2<C, ps_w2e<C>(), HS / 2>(Ly, F, item, pre);
  const bool fc2_thread = tid < 2 * C;
  const int n2 = tid % C, half = tid / C;
  __syncthreads();
  if (tid < kPsR * HS) {
    const int m = tid / HS, j = tid % HS;
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kPsW; ++q) v += part[(q * kPsR + m) * HS + j];
    v += Ly.b_fc1[j0 + j];
    sm.hs[m][j] = gelu_tanh(v);
  }
  __syncthreads();
  float* __restrict__ p2h = big;  // [2][kPsR][C] half sums (the fc1 partials are consumed)
  if (fc2_thread) {
    // the eight rows of GELU(fc1) as 16-byte broadcast reads of four hidden
    // columns, terms added in ascending hidden column (whole waves take this
    // branch: 2C is a multiple of 64, and half is uniform per wave)
    float p2[kPsR];
#pragma unroll
    for (int m = 0; m < kPsR; ++m) p2[m] = 0.f;
    const int jb = __builtin_amdgcn_readfirstlane(half) * (HS / 2);
#pragma unroll
    for (int j = 0; j < HS / 2; j += 4) {
#pragma unroll
      for (int m = 0; m < kPsR; ++m) {
        const f32x4 h4 = *reinterpret_cast<const f32x4*>(&sm.hs[m][jb + j]);
#pragma unroll
        for (int u = 0; u < 4; ++u) p2[m] = fmaf(h4[u], pre.w2v[j + u], p2[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < kPsR; ++m) p2h[(half * kPsR + m) * C + n2] = p2[m];
  }
  __syncthreads();
  for (int i = tid; i < kPsR * C; i += kPsT) {
    const int m = i / C, n = i % C, b = m0 + m;
    if (b < B) st_dev(a.P2 + ((int64_t)sl * B + b) * C + n, p2h[m * C + n] + p2h[(kPsR + m) * C + n]);
  }
}

// ---- the head: row -> ln_f, lm_head, the pick ----
template <int C, int VPL>
__device__ __forceinline__ void ps_head_item(const PsArgs& a, int row, PsHead& sm) {
  const int V = a.V;
  const int tid = ps_tid();
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int kc = C / kPsW;
  const int k0 = w * kc, k1 = k0 + kc;
  constexpr int kHB = 24 / VPL;
  float wv[kHB][VPL];
  auto load_batch = [&](int kb) {
#pragma unroll
    for (int j = 0; j < kHB; ++j) {
      const float* __restrict__ wr = a.wh + (int64_t)min(kb + j, C - 1) * V;
#pragma unroll
      for (int i = 0; i < VPL; ++i) wv[j][i] = ld_off<float>(wr, 4u * (unsigned)min(lane + 64 * i, V - 1));
    }
  };
  load_batch(k0);
  LnPar lp;
  if (w == 0) ln_load<C>(lp, a.lnfg, a.lnfb, lane);
  __syncthreads();  // the previous item's LDS reads are done
  for (int n = tid; n < C; n += kPsT) sm.xs[n] = ps_pending<C>(a, a.L[a.NL - 1].b_fc2, row, n);
  __syncthreads();
  if (w == 0) ps_ln_row<C>(sm.xs, lane, lp, a.epsf);
  __syncthreads();
  float acc[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) acc[i] = 0.f;
  for (int kb = k0; kb < k1; kb += kHB) {
    if (kb != k0) load_batch(kb);
#pragma unroll
    for (int j = 0; j < kHB; ++j) {
      if (kb + j < k1) {
        const float xv = sm.xs[kb + j];
#pragma unroll
        for (int i = 0; i < VPL; ++i) acc[i] = fmaf(xv, wv[j][i], acc[i]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) sm.part[w * 64 * VPL + lane + 64 * i] = acc[i];
  __syncthreads();
  if (w == 0) {
    Top2 t{-INFINITY, -INFINITY, V};
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (c < V) {
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < kPsW; ++q) v += sm.part[q * 64 * VPL + c];
        v += a.bh[c];
        scan(t, v, c, V);
      }
    }
    t = reduce_top2(t, V);
    if (lane == 0) {
      // pick_record's bookkeeping, with device-scope accesses for what the
      // next token step of the same launch reads
      const int L = ld_dev_i(a.lengths + row);
      st_dev_i(a.cur + row, (int64_t)t.i1);
      if (L >= 0 && L < a.Tmax) a.ids[(int64_t)L * a.B + row] = t.i1;
      const int s = L - a.t_base;
      if (a.margins != nullptr && s >= 0 && s < a.nm) a.margins[(int64_t)s * a.B + row] = t.m1 - t.m2;
      st_dev_i(a.lengths + row, L + 1);
      if (row == 0) st_dev_i(a.pos, ld_dev_i(a.pos) + 1);
    }
  }
}

template <int C, int VPL>
__global__ __launch_bounds__(kPsT) void decode_step_kernel(const PsArgs a) {
  static_assert(C % 64 == 0 && C <= kPsMaxC && 2 * C <= kPsT, "row width");
  __shared__ __align__(16) float lds[PsLds<C>::kTotal];
  __shared__ int flag;
  unsigned long long next = 0;  // threads 0 .. 63: the next barrier's target
  PsSmem& sm = *reinterpret_cast<PsSmem*>(lds);
  float* const big = lds + PsLds<C>::kSlabOff;
  // a step after a failed wait on this workspace does nothing
  if (threadIdx.x == 0)
    flag = __hip_atomic_load(a.bar + kBarErr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u;
  if (threadIdx.x < 64)
    next = __hip_atomic_load(reinterpret_cast<unsigned long long*>(a.bar + kBarBase), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) +
           gridDim.x;
  __syncthreads();
  if (!flag) return;
  const int na = ((a.B + kPsS - 1) / kPsS) * a.H;
  const int nb = ((a.B + kPsR - 1) / kPsR) * (a.F / ps_hs<C>());
  const int first = blockIdx.x;
  PreA pa;
  if (first < na) attn_prefetch<C>(a, 0, first, pa);
  // token steps x blocks as one loop (a loop nest here makes the compiler
  // keep more values live across stages)
  const int nq = a.steps * a.NL;
  for (int q = 0; q < nq; ++q) {
    const int l = q % a.NL;
    // the slab region is free: the last stage B's reads ended before the barrier
    if (PsLds<C>::kApart && first < nb) mlp_dma<C>(a.L[l], a.F, first, big);
    for (int it = first; it < na; it += gridDim.x) ps_attn_item<C>(a, l, it, sm.a, pa, it == first);
    {
      ps_arrive(a);
      // (after the arrival's workgroup barrier stage A's LDS reads are done,
      // so a slab that lies over them can be requested)
      if (!PsLds<C>::kApart && first < nb) mlp_dma<C>(a.L[l], a.F, first, big);
      if (!ps_wait(a, &flag, next)) return;
    }
    for (int it = first; it < nb; it += gridDim.x) ps_mlp_item<C>(a, l, it, sm.b, big, it == first);
    if (l + 1 == a.NL) {
      if (!ps_barrier(a, &flag, next)) return;
      for (int r = blockIdx.x; r < a.B; r += gridDim.x) ps_head_item<C, VPL>(a, r, sm.h);
      if (q + 1 == nq) break;
      // the next step reads the picks, lengths and position just written
    }
    // the next stage's first weights are requested after the arrival (the
    // scheduling barriers keep their loads from moving into the stage before,
    // where their registers would add to its own, or ahead of the arrival)
    {
      ps_arrive(a);
      __builtin_amdgcn_sched_barrier(0);
      if (first < na) attn_prefetch<C>(a, l + 1 == a.NL ? 0 : l + 1, first, pa);
      __builtin_amdgcn_sched_barrier(0);
      if (!ps_wait(a, &flag, next)) return;
    }
  }
  // every workgroup has passed every barrier: the counters' total stands at
  // the last target, the next launch's base
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(a.bar + kBarBase), next - gridDim.x,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void decode_reset_kernel(unsigned* bar) {
  for (int i = threadIdx.x; i < kBarBytes / 4; i += blockDim.x) bar[i] = 0u;
}

// workspace layout: barrier words, X0, X1, P1, P2 (each 256-byte aligned)
struct PsLayout {
  size_t x0, x1, p1, p2, total;
};
inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }
PsLayout ps_layout(int B, int C, int H, int F) {
  PsLayout L;
  const size_t row = (size_t)B * C * sizeof(float);
  size_t off = kBarBytes;
  L.x0 = off;
  off += al256(row);
  L.x1 = off;
  off += al256(row);
  L.p1 = off;
  off += al256((size_t)H * row);
  L.p2 = off;
  off += al256((size_t)(F / ps_hs_host(C)) * row);
  L.total = off;
  return L;
}

// the kernel instances: row width C in {128, 256, 384, 512} (index C/128 - 1)
// by logits per lane VPL in {2, 4} (V <= 128, V <= 256)
constexpr int kPsNC = 4, kPsNV = 2;
template <int C>
void ps_row(const void** k) {
  k[0] = reinterpret_cast<const void*>(&decode_step_kernel<C, 2>);
  k[1] = reinterpret_cast<const void*>(&decode_step_kernel<C, 4>);
}
const void* ps_kernel(int ci, int vi) {
  static const void* table[kPsNC][kPsNV];
  static std::once_flag once;
  std::call_once(once, [] {
    ps_row<128>(table[0]);
    ps_row<256>(table[1]);
    ps_row<384>(table[2]);
    ps_row<512>(table[3]);
  });
  return table[ci][vi];
}

// per device: compute units, resident workgroups per unit for each kernel
// instance, wall-clock rate (kHz), cooperative launch support
struct PsDev {
  bool init = false;
  int ncu = 0, coop = 0, rate_khz = 0;
  int per_cu[kPsNC][kPsNV] = {};
};
std::mutex g_ps_mu;
PsDev g_ps_dev[64];

int ps_device(PsDev& out) {
  int dev = 0;
  MTX_HIP(hipGetDevice(&dev));
  MTX_CHECK_ARG(dev >= 0 && dev < 64, "decode_step: device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_ps_mu);
  PsDev& d = g_ps_dev[dev];
  if (!d.init) {
    MTX_HIP(hipDeviceGetAttribute(&d.ncu, hipDeviceAttributeMultiprocessorCount, dev));
    MTX_HIP(hipDeviceGetAttribute(&d.coop, hipDeviceAttributeCooperativeLaunch, dev));
    MTX_HIP(hipDeviceGetAttribute(&d.rate_khz, hipDeviceAttributeWallClockRate, dev));
    for (int ci = 0; ci < kPsNC; ++ci)
      for (int vi = 0; vi < kPsNV; ++vi)
        MTX_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&d.per_cu[ci][vi], ps_kernel(ci, vi), kPsT, 0));
    d.init = true;
  }
  out = d;
  return MTX_OK;
}

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" size_t mtx_decode_step_workspace_bytes(int B, int C, int n_head, int F) {
  if (B < 1 || C < 1 || n_head < 1 || F < kPsHS) return 0;
  return ps_layout(B, C, n_head, F).total;
}

extern "C" int mtx_decode_step_f32(const mtx_decode_model* m, int steps, int64_t* cur, int64_t* ids,
                                   float* margins, int t_base, int n_margins, int* lengths, int64_t* pos,
                                   void* workspace, size_t workspace_bytes, int64_t wait_limit_us, void* stream) {
  MTX_CHECK_ARG(m != nullptr, "decode_step: null model");
  MTX_CHECK_ARG(steps >= 1, "decode_step: steps must be >= 1 (got %d)", steps);
  const int NL = m->n_layer, B = m->B, C = m->C, H = m->n_head, F = m->F, V = m->V, Tmax = m->Tmax;
  MTX_CHECK_SHAPE(NL >= 1 && NL <= kPsMaxL && B >= 1 && H >= 1 && H <= kPsMaxH && C == H * kPsD &&
                      C % 128 == 0 && F == 4 * C && V >= 1 && V <= kPsMaxV &&
                      Tmax >= 1 &&
                      Tmax <= kPsMaxT && (int64_t)B * Tmax * C < ((int64_t)1 << 40),
                  "decode_step: needs 1 <= n_layer <= %d, head size 64, C = 64 n_head in {128, 256, 384, %d}, F = 4C, "
                  "V <= %d, 1 <= Tmax <= %d (got n_layer=%d C=%d n_head=%d F=%d V=%d Tmax=%d)",
                  kPsMaxL, kPsMaxC, kPsMaxV, kPsMaxT, NL, C, H, F, V, Tmax);
  MTX_CHECK_ARG(m->tok_emb && m->pos_emb && m->layers && m->lnf_gamma && m->lnf_beta && m->w_head && m->b_head,
                "decode_step: null model pointer");
  MTX_CHECK_ARG(m->n_tok >= 1 && m->n_pos >= 1, "decode_step: empty embedding table");
  MTX_CHECK_ARG(std::isfinite(m->lnf_eps) && m->lnf_eps >= 0.f, "decode_step: eps must be finite and >= 0");
  for (int l = 0; l < NL; ++l) {
    const mtx_decode_layer& y = m->layers[l];
    MTX_CHECK_ARG(y.ln1_gamma && y.ln1_beta && y.w_qkv && y.b_qkv && y.w_out && y.b_out && y.ln2_gamma &&
                      y.ln2_beta && y.w_fc1 && y.b_fc1 && y.w_fc2 && y.b_fc2 && y.k_cache && y.v_cache,
                  "decode_step: null pointer in layer %d", l);
    MTX_CHECK_ARG(((uintptr_t)y.k_cache & 15u) == 0 && ((uintptr_t)y.v_cache & 15u) == 0 &&
                      ((uintptr_t)y.w_out & 15u) == 0,
                  "decode_step: layer %d caches and w_out must be 16-byte aligned", l);
    MTX_CHECK_ARG(std::isfinite(y.ln1_eps) && y.ln1_eps >= 0.f && std::isfinite(y.ln2_eps) && y.ln2_eps >= 0.f,
                  "decode_step: layer %d eps must be finite and >= 0", l);
  }
  MTX_CHECK_ARG(cur && ids && lengths && pos, "decode_step: cur, ids, lengths, pos: null pointer");
  MTX_CHECK_ARG(margins == nullptr || n_margins >= 1, "decode_step: n_margins must be >= 1 with a margin buffer");
  const PsLayout lay = ps_layout(B, C, H, F);
  MTX_CHECK_ARG(workspace != nullptr && ((uintptr_t)workspace & 255u) == 0 && workspace_bytes >= lay.total,
                "decode_step: needs a 256-byte aligned workspace of %zu bytes (got %zu)", lay.total,
                workspace_bytes);

  PsDev d;
  int rc = ps_device(d);
  if (rc) return rc;
  MTX_CHECK_ARG(d.coop != 0, "decode_step: the device does not support cooperative launches");
  const int ci = C / 128 - 1, vi = V <= 128 ? 0 : 1;
  const int resident = d.per_cu[ci][vi] * d.ncu;
  MTX_CHECK_SHAPE(resident >= 1, "decode_step: the kernel does not fit a compute unit");
  const int na = ((B + kPsS - 1) / kPsS) * H, nb = ((B + kPsR - 1) / kPsR) * (F / ps_hs_host(C));
  const int G = std::min(resident, std::max(std::max(na, nb), B));

  char* ws = static_cast<char*>(workspace);
  PsArgs a{};
  a.NL = NL; a.B = B; a.C = C; a.H = H; a.F = F; a.V = V; a.Tmax = Tmax;
  a.scale = 1.0f / std::sqrt((float)kPsD);
  a.tok = m->tok_emb; a.ntok = m->n_tok;
  a.posw = m->pos_emb; a.npos = m->n_pos;
  a.lnfg = m->lnf_gamma; a.lnfb = m->lnf_beta; a.epsf = m->lnf_eps;
  a.wh = m->w_head; a.bh = m->b_head;
  a.cur = cur; a.ids = ids; a.margins = margins; a.t_base = t_base; a.nm = n_margins;
  a.lengths = lengths; a.pos = pos;
  a.X0 = reinterpret_cast<float*>(ws + lay.x0);
  a.X1 = reinterpret_cast<float*>(ws + lay.x1);
  a.P1 = reinterpret_cast<float*>(ws + lay.p1);
  a.P2 = reinterpret_cast<float*>(ws + lay.p2);
  a.bar = reinterpret_cast<unsigned*>(ws);
  const int64_t us = wait_limit_us == 0 ? 2000000 : wait_limit_us;
  a.limit = us < 0 ? -1 : us * (int64_t)d.rate_khz / 1000;
  for (int l = 0; l < NL; ++l) a.L[l] = m->layers[l];
  a.steps = steps;

  void* args[] = {&a};
  hipStream_t st = static_cast<hipStream_t>(stream);
  MTX_HIP(hipLaunchCooperativeKernel(ps_kernel(ci, vi), dim3(G), dim3(kPsT), args, 0, st));
  MTX_LAUNCHED();
  return MTX_OK;
}

extern "C" int mtx_decode_step_status(const void* workspace, void* stream) {
  MTX_CHECK_ARG(workspace != nullptr, "decode_step_status: null workspace");
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned err = 0;
  MTX_HIP(hipMemcpyAsync(&err, static_cast<const unsigned*>(workspace) + kBarErr, sizeof(unsigned),
                         hipMemcpyDeviceToHost, st));
  MTX_HIP(hipStreamSynchronize(st));
  if (err != 0u)
    return fail(MTX_ERR_HIP,
                "decode_step: a grid-wide wait ran out; that step's results are incomplete and later steps "
                "on this workspace did nothing (mtx_decode_step_reset clears it)");
  return MTX_OK;
}

extern "C" int mtx_decode_step_reset(void* workspace, void* stream) {
  MTX_CHECK_ARG(workspace != nullptr, "decode_step_reset: null workspace");
  hipLaunchKernelGGL(decode_reset_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<unsigned*>(workspace));
  MTX_LAUNCHED();
  return MTX_OK;
}
