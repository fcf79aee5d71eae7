// Fused causal multi-head attention for gfx950 (MI355X): forward, and a
// deterministic two-pass backward.
//
// Replaces the reference's composed attention sub-graph, transformer.py:36-44
// (q @ k^T, * 1/sqrt(D), + triu(-1e9), F.softmax, @ v) and the backward
// closures of those nodes (tensor.py:210-218, 152-156, 115-119;
// functional.py:69-73).
//
// Design (256-thread workgroups = 4 wave64s, 16x16 MFMA tiles; the bf16
// dK/dV pass takes MTX_DKDV_WAVES waves):
//  * "Transposed" products.  The forward and the dQ pass compute S^T = K Q^T, so
//    a lane's accumulator column is one query: lane l owns query l%16 and keys
//    4*(l/16)+r of each 16-key sub-tile.  Row max / row sum then need only two
//    lane swaps (v_permlane16/32_swap), the O rescale is per lane, and the probabilities are already
//    in the B-operand layout of O^T += V^T P^T (no LDS round trip for P).
//  * The dK/dV pass computes S = Q K^T (lane owns a key) so that P and dS feed
//    dV^T += dO^T P and dK^T += Q^T dS straight from registers, accumulating
//    dK/dV for the workgroup's key block in registers over all query tiles.
//  * dQ is a separate query-outer pass (recomputes S and dP) instead of fp32
//    atomics: deterministic, and no dQ workspace traffic.
//  * K/V (or Q/dO) tiles are staged through LDS row-major: bf16 tiles by
//    direct global -> LDS loads (16 bytes per lane, XOR-permuted 16-byte
//    chunks; two buffers, one barrier per tile), fp32 tiles through registers
//    into padded rows (D <= 64: one buffer, two barriers per tile); operands
//    that need the transposed tile are read with
//    gfx950's transposing LDS load (ds_read_b64_tr_b16), so each tile is
//    stored once.
//  * Causal: tiles above the diagonal are skipped at workgroup and wave level;
//    only diagonal tiles pay for the per-element mask.  Blocks are issued
//    longest-first and all blocks of one (b,h) go to one XCD (workgroup ids are
//    dealt round-robin over the 8 XCDs), so K/V re-reads hit that XCD's L2.
#include "mtx_common.h"

#include <atomic>
#include <cmath>
#include <mutex>
#include <type_traits>

// fp32, D <= 64: one tile buffer (staged through registers, two barriers
// per tile) halves the LDS per workgroup (35 KB), so twice as many
// workgroups share a CU; measured 9% faster than two buffers at C1
#ifndef MTX_F32_NBUF1
#define MTX_F32_NBUF1 1
#endif
// waves per SIMD the dQ kernel is compiled for (bf16, D <= 64; fp32 D = 128:
// 1, for its accumulators; others 2)
#ifndef MTX_DQ_WAVES
#define MTX_DQ_WAVES 3
#endif
// waves per SIMD the forward kernel is compiled for (bf16, D <= 64; fp32
// D = 128: 1; others 2)
#ifndef MTX_FWD_WAVES
#define MTX_FWD_WAVES 4
#endif
// 1: the dK/dV tile body is instantiated twice (masked diagonal tiles,
// unmasked interior tiles); 0: one body with a run-time mask test
// split-bf16 fp32 passes at D = 64: one wave per SIMD (the whole register
// file) for dK/dV and dQ, and the 16-key / 16-query sub-blocks per wave
#ifndef MTX_X3_DKDV_WAVES1
#define MTX_X3_DKDV_WAVES1 1
#endif
#ifndef MTX_X3_DQ_WAVES1
#define MTX_X3_DQ_WAVES1 1
#endif
#ifndef MTX_X3_NK
#define MTX_X3_NK 2
#endif
#ifndef MTX_X3_NQ
#define MTX_X3_NQ 2
#endif
#ifndef MTX_DKDV_SPLIT
#define MTX_DKDV_SPLIT 1
#endif

namespace mtx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;

struct Str3 {
  int64_t b, h, t;  // element strides; the d stride is 1
};

struct FwdArgs {
  const void* q; Str3 sq;
  const void* k; Str3 sk;
  const void* v; Str3 sv;
  void* o; Str3 so;
  float* lse;
  int B, H, Tq, Tk;
  float scale;
  int causal;
  // attention dropout (keep == nullptr: none): keep[(bh*Tq + i)*kld + j] != 0
  // keeps P[i][j], scaled by kscale = 1/(1-p); kld is a multiple of 4
  const uint8_t* keep;
  int64_t kld;
  float kscale;
};

struct BwdArgs {
  const void* q; Str3 sq;
  const void* k; Str3 sk;
  const void* v; Str3 sv;
  const void* o; Str3 so;
  const void* dout; Str3 sdo;
  const float* lse;
  float* delta;
  float* dq; Str3 sdq;
  float* dk; Str3 sdk;
  float* dv; Str3 sdv;
  int B, H, Tq, Tk;
  float scale;
  int causal;
  int accumulate;
  const uint8_t* keep;  // attention dropout, as in FwdArgs
  int64_t kld;
  float kscale;
};

// Work mapping: block id -> (tile index, bh).  Blocks of one bh share an XCD
// (xcd = id % 8) and, for causal, the heaviest tiles are issued first.
__device__ __forceinline__ void map_block(int bid, int ntile, int BH, bool heavy_last,
                                          int& tile, int& bh) {
  int rank;
  if ((BH & 7) == 0) {
    const int x = bid & 7, local = bid >> 3, per = BH >> 3;
    bh = (local % per) * 8 + x;
    rank = local / per;
  } else {
    bh = bid % BH;
    rank = bid / BH;
  }
  tile = heavy_last ? (ntile - 1 - rank) : rank;
}

// ---------------------------------------------------------------------------
// LDS tile staging
// ---------------------------------------------------------------------------
// A tile in flight: global -> registers (fetch) and registers -> LDS (put,
// row-major with row stride ld), so the next tile's global loads overlap the
// current tile's MFMA work.
template <typename T, int R, int D>
struct TileRegs {
  static constexpr int V = Elem<T>::kVec;
  static constexpr int CPR = D / V;                           // 16-byte chunks per row
  static constexpr int NCH = R * CPR;                         // chunks per tile
  static constexpr int PER = (NCH + kThreads - 1) / kThreads;  // chunks per thread
  uint4 r[PER];

  // Rows >= nrows read as zero.  The tile's first row is a wave-uniform
  // pointer and each lane adds a 32-bit offset (row strides are < 2^24
  // elements, checked on the host); whole tiles take a branch without guards.
  __device__ __forceinline__ void fetch(const T* __restrict__ g, int64_t ts, int r0, int nrows, int tid) {
    const T* __restrict__ base = g + (int64_t)r0 * ts;
    const int its = (int)ts;
    if (r0 + R <= nrows) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = tid + i * kThreads;
        if (NCH % kThreads != 0 && c >= NCH) continue;
        const int rr = c / CPR, cc = c % CPR;
        r[i] = *reinterpret_cast<const uint4*>(base + rr * its + cc * V);
      }
    } else {
      const int nrel = nrows - r0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = tid + i * kThreads;
        const int rr = c / CPR, cc = c % CPR;
        uint4 v0 = make_uint4(0u, 0u, 0u, 0u);
        if ((NCH % kThreads == 0 || c < NCH) && rr < nrel)
          v0 = *reinterpret_cast<const uint4*>(base + rr * its + cc * V);
        r[i] = v0;
      }
    }
  }

  __device__ __forceinline__ void put(T* __restrict__ buf, int ld, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * kThreads;
      if (NCH % kThreads != 0 && c >= NCH) continue;
      const int rr = c / CPR, cc = c % CPR;
      *reinterpret_cast<uint4*>(buf + rr * ld + cc * V) = r[i];
    }
  }
};

// LDS tile layout.  bf16 tiles have unpadded rows whose 16-byte chunks are
// permuted per row (chunk c of row r at chunk c ^ swz(r)), so that the two
// fragment read patterns (16-byte reads of 16 consecutive rows at one column;
// 8-byte transposing reads of 4-row x 16-column blocks) spread over the LDS
// banks and a wave's 1 KiB direct load (TileDma) is one contiguous run of
// rows.  swz has period 16 in r, so a fragment's offset inside a 16-row block
// is a per-lane constant.  fp32 tiles use padded rows (register staging).
template <typename T, int D>
struct Lay {
  static constexpr bool DIRECT = sizeof(T) == 2;  // global -> LDS loads
  static constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;              // chunks per row
  static constexpr int LD = DIRECT ? D : D + 4;    // row stride (elements)
  __host__ __device__ static constexpr int swz(int r) {
    return ((((r >> 1) << 1) + ((r >> 3) & 1)) & 7) & (CPR - 1);
  }
  // element offset of (r, col); an access must not cross a 16-byte chunk
  __host__ __device__ static constexpr int at(int r, int col) {
    if constexpr (DIRECT) return r * LD + ((((col / EPC) ^ swz(r)) * EPC) | (col % EPC));
    else return r * LD + col;
  }
};

// ---------------------------------------------------------------------------
// fp32 attention on the bf16 matrix cores (T = f32x3_t)
// ---------------------------------------------------------------------------
// The kernels run on fp32 data the way the GEMMs' default mode does: each
// fp32 operand value x is split into x0 = bf16(x), x1 = bf16(x - x0),
// x2 = bf16(x - x0 - x1) (round to nearest even, each difference exact), so
// x = x0 + x1 + x2 to 2^-24 |x|, and a product is the sum of the six piece
// products of weight >= 2^-16 (x2y0, x1y1, x0y2, x1y0, x0y1, x0y0), each
// exact in fp32 and added into the fp32 accumulator by the matrix core: six
// v_mfma_f32_16x16x32_bf16 (6 x 16 cycles) do the work of eight
// v_mfma_f32_16x16x4_f32 (8 x 32 cycles).  Tiles are fetched as fp32 into
// registers and split while stored, as three bf16 planes in the bf16 kernels'
// LDS layout; the register operands (the pre-scaled Q or K, dO, V) and the
// probabilities P and dS are split the same way.  Global data stays fp32.
struct f32x3_t {};
struct Frag3 {
  bf16x8 p[3];
};
}  // namespace
// (an explicit specialisation lives in the template's own namespace)
template <> struct Mfma<f32x3_t> {
  static constexpr int KI = 32;
  static constexpr int KPL = 8;
  typedef Frag3 frag;
  __device__ __forceinline__ static f32x4 mma(const frag& a, const frag& b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[2], b.p[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[1], b.p[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[0], b.p[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[1], b.p[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[0], b.p[1], c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.p[0], b.p[0], c, 0, 0, 0);
  }
};
namespace {
template <typename T> constexpr bool is_x3() { return std::is_same<T, f32x3_t>::value; }
// element type in global memory and in LDS tiles
template <typename T> struct GEl { using type = T; };
template <> struct GEl<f32x3_t> { using type = float; };
template <typename T> struct LEl { using type = T; };
template <> struct LEl<f32x3_t> { using type = bf16_t; };
// planes per LDS tile; every tile of these kernels has 64 rows
template <typename T> constexpr int planes() { return is_x3<T>() ? 3 : 1; }
constexpr int kTileRows = 64;
// the bf16 kernels' swizzled row layout, filled through registers
template <int D>
struct Lay<f32x3_t, D> : Lay<bf16_t, D> {
  static constexpr bool DIRECT = false;
  static constexpr int PS = kTileRows * D;  // plane stride (bf16 elements)
};

// eight fp32 values -> three bf16x8 pieces
__device__ __forceinline__ Frag3 split8(const float (&v)[8]) {
  Frag3 f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = (__bf16)v[e];
    const float r1 = v[e] - (float)h;
    const __bf16 m = (__bf16)r1;
    f.p[0][e] = h;
    f.p[1][e] = m;
    f.p[2][e] = (__bf16)(r1 - (float)m);
  }
  return f;
}

// an fp32 tile of R rows through registers into three bf16 planes (the
// fetch of TileRegs<float>; the put splits every value)
template <int R, int D>
struct TileRegsX3 {
  using LY = Lay<bf16_t, D>;
  static constexpr int CPR = D / 4;                            // 16-byte fp32 chunks per row
  static constexpr int NCH = R * CPR;
  static constexpr int PER = (NCH + kThreads - 1) / kThreads;
  f32x4 r[PER];
  __device__ __forceinline__ void fetch(const float* __restrict__ g, int64_t ts, int r0, int nrows, int tid) {
    const float* __restrict__ base = g + (int64_t)r0 * ts;
    const int its = (int)ts;
    const int nrel = nrows - r0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * kThreads;
      const int rr = c / CPR, cc = c % CPR;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if ((NCH % kThreads == 0 || c < NCH) && (r0 + R <= nrows || rr < nrel))
        v = *reinterpret_cast<const f32x4*>(base + rr * its + cc * 4);
      r[i] = v;
    }
  }
  __device__ __forceinline__ void put(bf16_t* __restrict__ buf, int, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * kThreads;
      if (NCH % kThreads != 0 && c >= NCH) continue;
      const int rr = c / CPR, cc = c % CPR;
      const int o = LY::at(rr, 4 * cc);
      uint2 h, m, l;
      h.x = pack_bf2(r[i][0], r[i][1]);
      h.y = pack_bf2(r[i][2], r[i][3]);
      float d0 = r[i][0] - __uint_as_float(h.x << 16), d1 = r[i][1] - __uint_as_float(h.x & 0xffff0000u);
      float d2 = r[i][2] - __uint_as_float(h.y << 16), d3 = r[i][3] - __uint_as_float(h.y & 0xffff0000u);
      m.x = pack_bf2(d0, d1);
      m.y = pack_bf2(d2, d3);
      d0 -= __uint_as_float(m.x << 16);
      d1 -= __uint_as_float(m.x & 0xffff0000u);
      d2 -= __uint_as_float(m.y << 16);
      d3 -= __uint_as_float(m.y & 0xffff0000u);
      l.x = pack_bf2(d0, d1);
      l.y = pack_bf2(d2, d3);
      *reinterpret_cast<uint2*>(buf + o) = h;
      *reinterpret_cast<uint2*>(buf + Lay<f32x3_t, D>::PS + o) = m;
      *reinterpret_cast<uint2*>(buf + 2 * Lay<f32x3_t, D>::PS + o) = l;
    }
  }
};
template <typename T, int R, int D> struct TileRegsSel { using type = TileRegs<T, R, D>; };
template <int R, int D> struct TileRegsSel<f32x3_t, R, D> { using type = TileRegsX3<R, D>; };

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// bf16 tile of R rows staged by direct global -> LDS loads through a buffer
// resource (buffer_load_dwordx4 ... lds: lane i of a wave writes bytes
// [16i, 16i+16) of the wave's 1 KiB destination), so no registers hold the
// next tile.  Each lane loads the global chunk that belongs at its LDS
// position, at a 32-bit byte offset that is the same for every tile; the
// resource (scalar registers) starts at the tile's first row and spans the
// rows left in the (b,h) slice, so rows >= nrows read as zeros (finite data
// the kernels mask or weight by 0) with no per-lane test or address math.
// Completion: s_waitcnt vmcnt(0) by every wave, then a barrier.
template <typename T, int R, int D, int NW = kWaves>
struct TileDma {
  using LY = Lay<T, D>;
  static constexpr int NI = R * LY::CPR / 64;     // wave-loads per tile
  static constexpr int PW = (NI + NW - 1) / NW;   // per wave
  const T* base;
  int64_t ts;
  int nrows;
  uint32_t off[PW];  // byte offsets of this lane's chunks inside a tile

  // base: row 0 of the (b,h) slice; ts: its row stride (elements); the host
  // has checked nrows * ts * sizeof(T) < 2^31
  __device__ __forceinline__ void init(const T* b, int64_t t, int n, int wid, int lane) {
    base = b;
    ts = t;
    nrows = n;
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int c = (wid + j * NW) * 64 + lane;
      const int row = c / LY::CPR, pch = c % LY::CPR;
      off[j] = (uint32_t)(row * (int)t + (pch ^ LY::swz(row)) * LY::EPC) * (uint32_t)sizeof(T);
    }
  }
  __device__ __forceinline__ void issue(int r0, T* buf, int wid) const {
    // device pass only: the host pass would otherwise drop the stubs of the
    // kernels that use the AMDGPU buffer-resource type
#if defined(__HIP_DEVICE_COMPILE__)
    const int bytes = (nrows - r0) * (int)ts * (int)sizeof(T);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + (int64_t)r0 * ts), (short)0, bytes, 0x00020000);
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int ins = wid + j * NW;
      if (NI % NW != 0 && ins >= NI) continue;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(buf + ins * 64 * LY::EPC), 16, off[j], 0, 0, 0);
    }
#endif
  }
};

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Attention dropout (the reference's Dropout on the softmax output,
// layers.py:115-122 applied at transformer.py:43): P[i][j] is multiplied by
// keep[i][j] * kscale.  keep4: the keep bytes of keys j0 .. j0+3 of one
// query row as one dword (j0 % 4 == 0 and kld % 4 == 0 keep it aligned and
// inside the row); zf: the factor for byte r of such a word.
__device__ __forceinline__ uint32_t keep4(const uint8_t* __restrict__ keep, int64_t row_off, int j0, int64_t kld) {
  return j0 < kld ? *reinterpret_cast<const uint32_t*>(keep + row_off + j0) : 0u;
}
__device__ __forceinline__ float zf(uint32_t w, int r, float ks) { return ((w >> (8 * r)) & 0xffu) ? ks : 0.f; }

// Reductions over the 4 lanes l, l^16, l^32, l^48 of a wave64 with the gfx950
// lane swaps: v_permlane16_swap / v_permlane32_swap leave {v[l], v[l^16]}
// (resp. l^32) in the two results, in some order, on every lane, so a
// commutative op of the two needs no lane select.  Every lane of the group
// gets the same bits.
// v_max_f32 without the NaN-quieting copies fmaxf adds for operands that come
// from lane moves (the scores are never NaN for valid inputs)
__device__ __forceinline__ float vmax(float x, float y) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
  return r;
}
__device__ __forceinline__ float max4l(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4l(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ---------------------------------------------------------------------------
// MFMA operand fragments
// ---------------------------------------------------------------------------
// Contraction over the head dim uses the "quarter" k-map: lane group g covers
// d in [g*D/4, (g+1)*D/4), chunk kc covers KPL consecutive d of that quarter.
template <typename T, int D>
struct DMap {
  static constexpr int QPL = D / 4;
  static constexpr int KPL = Mfma<T>::KPL;
  static constexpr int KC = (QPL + KPL - 1) / KPL;
};

// the 8 fp32 values of the bf16 quarter-map fragment kc of a global row
// (D = 16: 4 values, then zeros)
template <int D>
__device__ __forceinline__ void load8(const float* __restrict__ p, int g, int kc, float (&v)[8]) {
  constexpr int QPL = D / 4;
  const f32x4 a = *reinterpret_cast<const f32x4*>(p + g * QPL + 8 * kc);
  const f32x4 b = QPL >= 8 ? *reinterpret_cast<const f32x4*>(p + g * QPL + 8 * kc + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = a[e];
    v[e + 4] = b[e];
  }
}

// Fragment of a row stored row-major (in LDS or global): row pointer p.
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag dfrag(const typename GEl<T>::type* __restrict__ p, int g, int kc) {
  constexpr int QPL = D / 4;
  if constexpr (is_x3<T>()) {
    float v[8];
    load8<D>(p, g, kc, v);
    return split8(v);
  } else if constexpr (sizeof(T) == 4) {
    return p[g * QPL + kc];
  } else if constexpr (QPL >= 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(p + g * QPL + 8 * kc);
    return __builtin_bit_cast(bf16x8, u);
  } else {  // D == 16: 4 real elements, 4 zeros
    const uint2 u = *reinterpret_cast<const uint2*>(p + g * QPL);
    const uint4 w = make_uint4(u.x, u.y, 0u, 0u);
    return __builtin_bit_cast(bf16x8, w);
  }
}

// Transposed operand (ltfrag below): A operand X^T[d][j] for k-step s over the
// j (key or query) dimension of a row-major LDS tile X[j][d], for
// d = 16*dt + n, where the matching B operand comes from C-layout
// accumulators (see pfrag).
//   fp32: step s covers j = 16*(s/4) + 4g + (s%4): one scalar read.
//   bf16: step s covers j = 32s + 16*(e/4) + 4g + (e%4), e = 0..7, read with
//   two gfx950 transposing LDS loads (ds_read_b64_tr_b16).  Within each
//   16-lane group, element i of lane k's result is element (k%4) of the 8-byte
//   chunk addressed by lane 4i + k/4 of the group, so lane (g, n) addresses
//   X[32s + 4g + n/4][16dt + 4(n%4)] (and 16 rows further for e = 4..7) and
//   receives X[32s + 4g + i][16dt + n], i = 0..3.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Fragment reads from an LDS tile in the Lay<T, D> layout.  LaneOffs::d(kc):
// the lane's offset of the "quarter map" fragment kc inside a 16-row block
// (row n); LaneOffs::t(dt): the lane's offset of the transposed operand for
// d-block dt.  With the swizzle the offsets for other kc / dt differ from the
// first only in bits below the row base, by xor.
template <typename T, int D>
struct LaneOffs {
  using LY = Lay<T, D>;
  static constexpr int QPL = D / 4;
  int d0, t0;
  __device__ __forceinline__ LaneOffs(int n, int g) {
    d0 = LY::at(n, g * QPL);
    if constexpr (sizeof(T) == 4) t0 = LY::at(4 * g, n);
    else t0 = LY::at(4 * g + (n >> 2), 4 * (n & 3));
  }
  __device__ __forceinline__ int d(int kc) const {
    if constexpr (LY::DIRECT) return d0 ^ (kc * (sizeof(T) == 4 ? 1 : 8));
    else return d0 + kc * (sizeof(T) == 4 ? 1 : 8);
  }
  __device__ __forceinline__ int t(int dt) const {
    if constexpr (LY::DIRECT) return t0 ^ (16 * dt);
    else return t0 + 16 * dt;
  }
};

template <int D>
struct LaneOffs<f32x3_t, D> : LaneOffs<bf16_t, D> {
  __device__ __forceinline__ LaneOffs(int n, int g) : LaneOffs<bf16_t, D>(n, g) {}
};

template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag lfrag(const typename LEl<T>::type* __restrict__ p) {
  if constexpr (is_x3<T>()) {
    constexpr int PS = Lay<f32x3_t, D>::PS;
    Frag3 f;
#pragma unroll
    for (int k = 0; k < 3; ++k) f.p[k] = lfrag<bf16_t, D>(p + k * PS);
    return f;
  } else if constexpr (sizeof(T) == 4) {
    return *p;
  } else if constexpr (D / 4 >= 8) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
  } else {  // D == 16: 4 real elements, 4 zeros
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return __builtin_bit_cast(bf16x8, make_uint4(u.x, u.y, 0u, 0u));
  }
}

// transposed operand for k-step s; `to` = LaneOffs::t(dt)
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag ltfrag(const typename LEl<T>::type* __restrict__ buf, int s, int to) {
  constexpr int LD = Lay<T, D>::LD;
  if constexpr (is_x3<T>()) {
    constexpr int PS = Lay<f32x3_t, D>::PS;
    Frag3 f;
#pragma unroll
    for (int k = 0; k < 3; ++k) f.p[k] = ltfrag<bf16_t, D>(buf + k * PS, s, to);
    return f;
  } else if constexpr (sizeof(T) == 4) {
    return buf[(16 * (s >> 2) + (s & 3)) * LD + to];
  } else {
    const T* p = buf + 32 * s * LD + to;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 16 * LD));
    const uint2 ul = __builtin_bit_cast(uint2, lo), uh = __builtin_bit_cast(uint2, hi);
    return __builtin_bit_cast(bf16x8, make_uint4(ul.x, ul.y, uh.x, uh.y));
  }
}

// Operand fragment multiplied by c (rounded back to T).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag scale_frag(typename Mfma<T>::frag f, float c) {
  if constexpr (sizeof(T) == 4) {
    return f * c;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (__bf16)((float)f[e] * c);
    return f;
  }
}

// Fragment of a global row multiplied by c: for T = f32x3_t the product is
// formed in fp32 and then split (scaling the pieces would round each).
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::frag dfrag_scaled(const typename GEl<T>::type* __restrict__ p, int g,
                                                               int kc, float c) {
  if constexpr (is_x3<T>()) {
    float v[8];
    load8<D>(p, g, kc, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= c;
    return split8(v);
  } else {
    return scale_frag<T>(dfrag<T, D>(p, g, kc), c);
  }
}

// acc + sum of the elements of an operand fragment (bf16: v_dot2 with ones).
template <typename T>
__device__ __forceinline__ float frag_sum(typename Mfma<T>::frag f, float acc) {
  if constexpr (sizeof(T) == 4) {
    return acc + f;
  } else {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const bf16x2 pr = {f[e], f[e + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
    }
    return acc;
  }
}

// B operand from C-layout accumulators c[j16] (16x16 sub-tiles along j), step s.
template <typename T, int NJ16>
__device__ __forceinline__ typename Mfma<T>::frag pfrag(const f32x4 (&c)[NJ16], int s) {
  if constexpr (is_x3<T>()) {
    const f32x4 a = c[2 * s], b = c[2 * s + 1];
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return split8(v);
  } else if constexpr (sizeof(T) == 4) {
    return c[s >> 2][s & 3];
  } else {
    const f32x4 a = c[2 * s], b = c[2 * s + 1];
    bf16x8 f;
    f[0] = (__bf16)a[0]; f[1] = (__bf16)a[1]; f[2] = (__bf16)a[2]; f[3] = (__bf16)a[3];
    f[4] = (__bf16)b[0]; f[5] = (__bf16)b[1]; f[6] = (__bf16)b[2]; f[7] = (__bf16)b[3];
    return f;
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* __restrict__ p, f32x4 v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4*>(p) = v;
  } else {
    uint2 u;
    u.x = pack_bf2(v[0], v[1]);
    u.y = pack_bf2(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = u;
  }
}

#ifndef MTX_GRAD_NT
#define MTX_GRAD_NT 1
#endif
// Gradients are written once and not read again by the attention passes:
// non-temporal stores, so they do not displace the q/k/v/o/dO tiles the
// other passes re-read from the caches
__device__ __forceinline__ void store_grad4(float* __restrict__ p, f32x4 v, bool acc) {
  if (acc) {
    const f32x4 old = *reinterpret_cast<const f32x4*>(p);
    v += old;
  }
#if MTX_GRAD_NT
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
#else
  *reinterpret_cast<f32x4*>(p) = v;
#endif
}


// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, int D, int NQ, bool DROP>
__global__ __launch_bounds__(kThreads, (sizeof(T) == 2 && D <= 64) ? MTX_FWD_WAVES : (D == 128 && sizeof(T) == 4 ? 1 : 2))
void attn_fwd_kernel(const FwdArgs a) {
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using DM = DMap<T, D>;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int KC = DM::KC;
  constexpr int DT = D / 16;
  constexpr int BQ = kWaves * NQ * 16;
  constexpr int BK = 64;
  constexpr int NS = BK / MF::KI;             // k-steps of the PV product per tile
  using LY = Lay<T, D>;
  constexpr int LD = LY::LD;  // LDS row stride
  constexpr int KSZ = BK * LD;
  using G = typename GEl<T>::type;   // element type in global memory
  using LT = typename LEl<T>::type;  // element type of the LDS tiles
  constexpr int NPLN = planes<T>();
  constexpr int NBUF = is_x3<T>() ? 1 : (sizeof(T) == 4 && D <= 64 && MTX_F32_NBUF1) ? 1 : (2 * KSZ * (int)sizeof(T) * 2 <= 80 * 1024 ? 2 : 1);
  static_assert(!LY::DIRECT || NBUF == 2, "direct tile loads need two buffers");
  // separate arrays per buffer, picked with compile-time parities: the
  // compiler then sees the direct loads into one buffer and the reads of the
  // other as disjoint and does not wait for the loads before the reads
  __shared__ __attribute__((aligned(16))) LT K0[KSZ * NPLN], V0[KSZ * NPLN];
  __shared__ __attribute__((aligned(16))) LT K1[NBUF == 2 ? KSZ * NPLN : 1], V1[NBUF == 2 ? KSZ * NPLN : 1];

  const int BH = a.B * a.H;
  const int nqb = (a.Tq + BQ - 1) / BQ;
  int qb, bh;
  map_block(blockIdx.x, nqb, BH, a.causal != 0, qb, bh);
  const int b = bh / a.H, h = bh % a.H;
  const G* __restrict__ qp = static_cast<const G*>(a.q) + b * a.sq.b + h * a.sq.h;
  const G* __restrict__ kp = static_cast<const G*>(a.k) + b * a.sk.b + h * a.sk.h;
  const G* __restrict__ vp = static_cast<const G*>(a.v) + b * a.sv.b + h * a.sv.h;
  G* __restrict__ op = static_cast<G*>(a.o) + b * a.so.b + h * a.so.h;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int n = lane & 15, g = lane >> 4;
  const int q0 = qb * BQ;
  const int qw0 = q0 + wid * NQ * 16;
  const int off = a.Tk - a.Tq;
  const float c = a.scale * kLog2e;

  // Q fragments (B operand of S^T = K Q^T), straight from global memory and
  // pre-multiplied by c = scale*log2(e), so the MFMA yields log2-unit scores
  frag qf[NQ][KC];
#pragma unroll
  for (int qs = 0; qs < NQ; ++qs) {
    const int row = qw0 + 16 * qs + n;
    const int rr = row < a.Tq ? row : a.Tq - 1;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      frag f = dfrag_scaled<T, D>(qp + (int64_t)rr * a.sq.t, g, kc, c);
      if (row >= a.Tq) f = frag{};
      qf[qs][kc] = f;
    }
  }

  // Online softmax against a reference m per query (log2 units) that moves
  // lazily: the S MFMA starts from -m, so it yields x = s*c - m and p =
  // exp2(x) directly.  m moves to the row max only on the row's first tile
  // or when a tile's max exceeds it by more than kTau (so p <= 2^kTau);
  // that path is taken by the whole wave (wave-uniform branch).  Any m gives
  // the same O = acc / l and lse = (m + log2 l) * ln2.
  constexpr float kTau = 8.f;
  f32x4 acc[NQ][DT];
  f32x4 cin[NQ];
  float m[NQ], l[NQ], lim[NQ];  // lim: -inf before the row's first key, kTau after
#pragma unroll
  for (int qs = 0; qs < NQ; ++qs) {
    m[qs] = -INFINITY;
    l[qs] = 0.f;
    lim[qs] = -INFINITY;
    cin[qs] = zero4();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[qs][dt] = zero4();
  }

  const int kend = a.causal ? min(a.Tk, q0 + BQ + off) : a.Tk;
  const int ntile = (kend + BK - 1) / BK;
  const LaneOffs<T, D> lo(n, g);
  TileDma<T, BK, D> kdma, vdma;  // bf16: direct global -> LDS
  typename TileRegsSel<T, BK, D>::type kreg, vreg;  // fp32: through registers
  if constexpr (LY::DIRECT) {
    kdma.init(kp, a.sk.t, a.Tk, wid, lane);
    vdma.init(vp, a.sv.t, a.Tk, wid, lane);
    if (ntile > 0) {
      kdma.issue(0, K0, wid);
      vdma.issue(0, V0, wid);
    }
  } else if (ntile > 0) {
    kreg.fetch(kp, a.sk.t, 0, a.Tk, tid);
    vreg.fetch(vp, a.sv.t, 0, a.Tk, tid);
  }
  // one key tile; P = buffer parity (for direct loads the loop below is
  // unrolled by two so that P is a compile-time constant)
  auto step = [&](auto par, const int it) {
    const int P = int(par) % NBUF;  // a constant for the unrolled (direct-load) loop
    const int PN = (P + 1) % NBUF;
    const int kb = it * BK;
    LT* __restrict__ Kb = P ? K1 : K0;
    LT* __restrict__ Vb = P ? V1 : V0;
    if constexpr (LY::DIRECT) {
      wait_dma();
    } else {
      if constexpr (NBUF == 1) __syncthreads();
      kreg.put(Kb, LD, tid);
      vreg.put(Vb, LD, tid);
    }
    __syncthreads();
    if (it + 1 < ntile) {
      if constexpr (LY::DIRECT) {
        kdma.issue(kb + BK, PN ? K1 : K0, wid);
        vdma.issue(kb + BK, PN ? V1 : V0, wid);
      } else {
        kreg.fetch(kp, a.sk.t, kb + BK, a.Tk, tid);
        vreg.fetch(vp, a.sv.t, kb + BK, a.Tk, tid);
      }
    }

    if (a.causal && kb > qw0 + NQ * 16 - 1 + off) return;  // nothing visible for this wave
    const bool need_mask = (kb + BK > a.Tk) || (a.causal && kb + BK - 1 > qw0 + off);

    // dropout keep bytes of this lane's query and keys kb + 16kt + 4g + 0..3,
    // requested before the score products so their latency overlaps them
    uint32_t kwd[NQ][4];
    if constexpr (DROP) {
#pragma unroll
      for (int qs = 0; qs < NQ; ++qs) {
        const int64_t ro = ((int64_t)bh * a.Tq + min(qw0 + 16 * qs + n, a.Tq - 1)) * a.kld;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kwd[qs][kt] = keep4(a.keep, ro, kb + 16 * kt + 4 * g, a.kld);
      }
    }

    f32x4 s[NQ][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      frag kf[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) kf[kc] = lfrag<T, D>(Kb + 16 * kt * LD + lo.d(kc));
#pragma unroll
      for (int qs = 0; qs < NQ; ++qs) {
        f32x4 t = cin[qs];
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) t = MF::mma(kf[kc], qf[qs][kc], t);
        s[qs][kt] = t;
      }
    }

    frag pf[NQ][NS];
#pragma unroll
    for (int qs = 0; qs < NQ; ++qs) {
      if (need_mask) {
        // key kb + 16kt + 4g + r is visible iff 16kt + r <= lim
        const int qi = qw0 + 16 * qs + n;
        int lim = a.Tk - 1 - kb - 4 * g;
        if (a.causal) lim = min(lim, qi + off - kb - 4 * g);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * kt + r > lim) s[qs][kt][r] = -INFINITY;
      }
      // a row's max exceeds lim iff one of its four lanes' maxima does, so
      // the lanes' own maxima decide the (wave-uniform) branch and the
      // cross-lane reduction runs only inside it
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[qs][kt][r]);
      if (__builtin_amdgcn_ballot_w64(mx > lim[qs]) != 0ull) {
        mx = max4l(mx);
        // move this lane's reference up by d (0 for lanes that keep theirs);
        // everything is updated in place
        const bool move = mx > lim[qs];
        const float d = move ? mx : 0.f;
        const bool fresh = m[qs] == -INFINITY;
        const float alpha = fresh ? 0.f : __builtin_amdgcn_exp2f(-d);
        m[qs] = fresh ? (move ? d : -INFINITY) : m[qs] + d;
        lim[qs] = m[qs] == -INFINITY ? -INFINITY : kTau;
        const float cm = m[qs] == -INFINITY ? 0.f : -m[qs];
        cin[qs] = f32x4{cm, cm, cm, cm};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[qs][kt] -= d;
        l[qs] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[qs][dt] *= alpha;
      }
      if constexpr (DROP) {
        // the row sum normalises the softmax before dropout; P V uses the
        // kept, rescaled probabilities
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pv = __builtin_amdgcn_exp2f(s[qs][kt][r]);
            l[qs] += pv;
            s[qs][kt][r] = pv * zf(kwd[qs][kt], r, a.kscale);
          }
#pragma unroll
        for (int st = 0; st < NS; ++st) pf[qs][st] = pfrag<T, 4>(s[qs], st);
      } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[qs][kt][r] = __builtin_amdgcn_exp2f(s[qs][kt][r]);
        if constexpr (is_x3<T>()) {
          // the fp32 probabilities (which the three pieces carry to 2^-24),
          // in the order the dropout variant adds them
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) l[qs] += s[qs][kt][r];
#pragma unroll
          for (int st = 0; st < NS; ++st) pf[qs][st] = pfrag<T, 4>(s[qs], st);
        } else {
#pragma unroll
          for (int st = 0; st < NS; ++st) {
            pf[qs][st] = pfrag<T, 4>(s[qs], st);
            l[qs] = frag_sum<T>(pf[qs][st], l[qs]);
          }
        }
      }
    }

#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const frag vf = ltfrag<T, D>(Vb, st, lo.t(dt));
#pragma unroll
        for (int qs = 0; qs < NQ; ++qs) acc[qs][dt] = MF::mma(vf, pf[qs][st], acc[qs][dt]);
      }
  };
  if constexpr (LY::DIRECT) {
    for (int it = 0; it < ntile; it += 2) {
      step(std::integral_constant<int, 0>{}, it);
      if (it + 1 < ntile) step(std::integral_constant<int, 1>{}, it + 1);
    }
  } else {
    for (int it = 0; it < ntile; ++it) step(it & 1, it);
  }

  // finalize: O = acc / l, lse = (m + log2 l) * ln2
#pragma unroll
  for (int qs = 0; qs < NQ; ++qs) {
    float lt = l[qs];
    lt = sum4l(lt);
    const int qi = qw0 + 16 * qs + n;
    if (qi < a.Tq) {
      const float inv = 1.0f / lt;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        store4<G>(op + (int64_t)qi * a.so.t + 16 * dt + 4 * g, acc[qs][dt] * inv);
      if (g == 0) a.lse[(int64_t)bh * a.Tq + qi] = (m[qs] + __log2f(lt)) * kLn2;
    }
  }
}

// ---------------------------------------------------------------------------
// backward, pass 0: delta[i] = sum_d dO[i,d] * O[i,d]
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_delta_kernel(const BwdArgs a) {
  const int64_t rows = (int64_t)a.B * a.H * a.Tq;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= rows) return;
  const int t = (int)(i % a.Tq);
  const int64_t bh = i / a.Tq;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const T* op = static_cast<const T*>(a.o) + b * a.so.b + h * a.so.h + (int64_t)t * a.so.t;
  const T* dp = static_cast<const T*>(a.dout) + b * a.sdo.b + h * a.sdo.h + (int64_t)t * a.sdo.t;
  constexpr int V = Elem<T>::kVec;
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < D / V; ++c) {
    const uint4 ou = *reinterpret_cast<const uint4*>(op + c * V);
    const uint4 du = *reinterpret_cast<const uint4*>(dp + c * V);
    const T* oe = reinterpret_cast<const T*>(&ou);
    const T* de = reinterpret_cast<const T*>(&du);
#pragma unroll
    for (int e = 0; e < V; ++e) sum = fmaf(Elem<T>::to_f(oe[e]), Elem<T>::to_f(de[e]), sum);
  }
  a.delta[i] = sum;
}

// ---------------------------------------------------------------------------
// one-pass backward, preparation: delta[i] = sum_d dO[i,d] O[i,d] and, unless
// the gradients accumulate, dq[i,:] = 0 (the one-pass dK/dV/dQ kernel adds
// into dq).  Four lanes per row, each summing D/4 consecutive products with
// fmaf in order, then (s0 + s1) + (s2 + s3): the dQ pass's order (its lane
// quarters and v_permlane swaps), so both structures see the same delta.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_prep_kernel(const BwdArgs a) {
  constexpr int QPL = D / 4;  // elements per lane
  const int64_t rows = (int64_t)a.B * a.H * a.Tq;
  const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t i = gid >> 2;
  const int c = (int)(gid & 3);
  const bool ok = i < rows;
  float sum = 0.f;
  int b = 0, h = 0, t = 0;
  if (ok) {
    t = (int)(i % a.Tq);
    const int64_t bh = i / a.Tq;
    b = (int)(bh / a.H);
    h = (int)(bh % a.H);
    const T* op = static_cast<const T*>(a.o) + b * a.so.b + h * a.so.h + (int64_t)t * a.so.t + c * QPL;
    const T* dp = static_cast<const T*>(a.dout) + b * a.sdo.b + h * a.sdo.h + (int64_t)t * a.sdo.t + c * QPL;
    constexpr int NW = QPL * (int)sizeof(T) / 8;  // 8-byte words per lane
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint2 ou = reinterpret_cast<const uint2*>(op)[w];
      const uint2 du = reinterpret_cast<const uint2*>(dp)[w];
      const T* oe = reinterpret_cast<const T*>(&ou);
      const T* de = reinterpret_cast<const T*>(&du);
#pragma unroll
      for (int e = 0; e < 8 / (int)sizeof(T); ++e) sum = fmaf(Elem<T>::to_f(oe[e]), Elem<T>::to_f(de[e]), sum);
    }
  }
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  if (ok) {
    if (c == 0) a.delta[i] = sum;
    if (!a.accumulate) {
      float* dq = a.dq + b * a.sdq.b + h * a.sdq.h + (int64_t)t * a.sdq.t + c * QPL;
#pragma unroll
      for (int j = 0; j < QPL; j += 4) *reinterpret_cast<f32x4*>(dq + j) = zero4();
    }
  }
}

// ---------------------------------------------------------------------------
// backward, pass 1: dK, dV (key-outer).  Each wave owns NK*16 keys.
// ---------------------------------------------------------------------------
// waves per workgroup of the bf16 dK/dV pass (they share each Q/dO tile)
#ifndef MTX_DKDV_WAVES
#define MTX_DKDV_WAVES 4
#endif
template <typename T>
constexpr int dkdv_waves() { return sizeof(T) == 2 ? MTX_DKDV_WAVES : kWaves; }

// FQ (one-pass backward, bf16): the pass also produces dQ.  Each tile's dS
// (bf16, the operand the dK product uses) is stored transposed in LDS (rows:
// the block's 128 keys, columns: the tile's 64 queries); after a barrier
// every wave multiplies it with the block's K (staged in LDS once) for its
// share of the dQ tile (dQ = scale dS K over the block's keys) and adds that
// share into dq with fp32 atomics.  dq must hold zeros (or the gradient to
// add to) and delta must be computed before the launch (attn_prep_kernel).
// Nothing of the dQ product stays in registers across tiles: the dK/dV pass
// already holds 2 waves per SIMD at the register file's limit.
// (An issue order that keeps all key blocks of a slice consecutively on one
// XCD, so that fewer slices take atomic adds at a time, measured the same.)
template <typename T, int D, int NK, bool DROP, bool FQ = false>
__global__ __launch_bounds__(64 * dkdv_waves<T>(), ((D == 128 && sizeof(T) == 4) || (is_x3<T>() && D == 64 && MTX_X3_DKDV_WAVES1)) ? 1 : 2) void attn_dkdv_kernel(const BwdArgs a) {
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using DM = DMap<T, D>;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int KC = DM::KC;
  constexpr int DT = D / 16;
  constexpr int NWV = dkdv_waves<T>();
  constexpr int BKV = NWV * NK * 16;
  constexpr int BQ = 64;
  constexpr int NS = BQ / MF::KI;
  using LY = Lay<T, D>;
  constexpr int LD = LY::LD;
  constexpr int RSZ = BQ * LD;
  using G = typename GEl<T>::type;   // element type in global memory
  using LT = typename LEl<T>::type;  // element type of the LDS tiles
  constexpr int NPLN = planes<T>();
  constexpr int NBUF = is_x3<T>() ? 1 : (sizeof(T) == 4 && D <= 64 && MTX_F32_NBUF1) ? 1 : (2 * RSZ * (int)sizeof(T) * 2 <= 80 * 1024 ? 2 : 1);
  static_assert(!LY::DIRECT || NBUF == 2, "direct tile loads need two buffers");
  // separate arrays per buffer, picked with compile-time parities (see the
  // forward kernel)
  __shared__ __attribute__((aligned(16))) LT Q0[RSZ * NPLN], D0[RSZ * NPLN];
  __shared__ __attribute__((aligned(16))) LT Q1[NBUF == 2 ? RSZ * NPLN : 1], D1[NBUF == 2 ? RSZ * NPLN : 1];
  // per query of the tile: -lse*log2(e) and -delta, the starting accumulators
  // of the S and dP MFMAs, so they yield log2(P) and dP - delta directly
  __shared__ __attribute__((aligned(16))) float L0[BQ], E0[BQ], L1[BQ], E1[BQ];
  // FQ: the tile's dS^T, and the block's K rows (row-major, the Q/dO tiles'
  // layout)
  static_assert(!FQ || (BF && !DROP && NWV == 4 && NK == 2 && D <= 64 && MF::KI == 32),
                "the one-pass backward is built for bf16, D <= 64, 4 waves x 32 keys");
  using LS = Lay<T, BQ>;  // dS^T rows: BQ bf16 each, swizzled like the Q/dO tiles
  __shared__ __attribute__((aligned(16))) LT S0[FQ ? BKV * BQ : 1], KS[FQ ? BKV * LD : 1];
  // bf16 two-pass, D <= 64: each wave's rows of dK, then of dV, staged for
  // whole-row stores (the one-pass and D = 128 kernels would lose their
  // second workgroup per CU to this LDS)
  constexpr bool GSTAGE = BF && !FQ && D <= 64;
  __shared__ __attribute__((aligned(16))) float GE[GSTAGE ? NWV * NK * 16 * D : 1];

  const int BH = a.B * a.H;
  const int nkb = (a.Tk + BKV - 1) / BKV;
  int kbk, bh;
  map_block(blockIdx.x, nkb, BH, false, kbk, bh);
  const int b = bh / a.H, h = bh % a.H;
  const G* __restrict__ qp = static_cast<const G*>(a.q) + b * a.sq.b + h * a.sq.h;
  const G* __restrict__ kp = static_cast<const G*>(a.k) + b * a.sk.b + h * a.sk.h;
  const G* __restrict__ vp = static_cast<const G*>(a.v) + b * a.sv.b + h * a.sv.h;
  const G* __restrict__ dop = static_cast<const G*>(a.dout) + b * a.sdo.b + h * a.sdo.h;
  const float* __restrict__ lsep = a.lse + (int64_t)bh * a.Tq;
  const float* __restrict__ delp = a.delta + (int64_t)bh * a.Tq;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int k0 = kbk * BKV;
  const int kw0 = k0 + wid * NK * 16;
  const int off = a.Tk - a.Tq;
  const float c = a.scale * kLog2e;


  f32x4 dka[NK][DT], dva[NK][DT];
#pragma unroll
  for (int ks = 0; ks < NK; ++ks)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) { dka[ks][dt] = zero4(); dva[ks][dt] = zero4(); }

  int qstart = a.causal ? max(0, k0 - off) : 0;
  qstart = (qstart / BQ) * BQ;
  const int ntile = qstart < a.Tq ? (a.Tq - qstart + BQ - 1) / BQ : 0;
  const LaneOffs<T, D> lo(n, g);
  TileDma<T, BQ, D, NWV> qdma, ddma;  // bf16: direct global -> LDS
  typename TileRegsSel<T, BQ, D>::type qreg, dreg;       // fp32: through registers
  if constexpr (LY::DIRECT) {
    qdma.init(qp, a.sq.t, a.Tq, wid, lane);
    ddma.init(dop, a.sdo.t, a.Tq, wid, lane);
  }
  float lse_r = 0.f, del_r = 0.f;
  // the next tile's loads: lse / delta (through registers, raw; converted
  // when stored, so the loads are not waited for here) first, so that waiting
  // for them never waits for the direct tile loads issued after them
  auto fetch = [&](int qt, LT* qdst, LT* ddst) {
    if (tid < BQ) {
      const int qi = min(qt + tid, a.Tq - 1);
      lse_r = lsep[qi];
      del_r = delp[qi];
    }
    if constexpr (LY::DIRECT) {
      qdma.issue(qt, qdst, wid);
      ddma.issue(qt, ddst, wid);
    } else {
      qreg.fetch(qp, a.sq.t, qt, a.Tq, tid);
      dreg.fetch(dop, a.sdo.t, qt, a.Tq, tid);
    }
  };
  if (ntile > 0) fetch(qstart, Q0, D0);
  if constexpr (FQ) {
    // the block's K rows into KS (waited for with the first tile)
    if (ntile > 0) {
      TileDma<T, BKV, D, NWV> kdma;
      kdma.init(kp, a.sk.t, a.Tk, wid, lane);
      kdma.issue(k0, KS, wid);
    }
  }
  // the K/V fragments are loaded after the first tile is requested, so both
  // latencies overlap (measured 1.5% faster at C3)
  // K and V fragments of this wave's keys (B operands of S = Q K^T, dP = dO V^T);
  // K pre-multiplied by c = scale*log2(e), so S comes out in log2 units
  frag kf[NK][KC], vf[NK][KC];
#pragma unroll
  for (int ks = 0; ks < NK; ++ks) {
    const int row = kw0 + 16 * ks + n;
    const int rr = row < a.Tk ? row : a.Tk - 1;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      frag fk = dfrag_scaled<T, D>(kp + (int64_t)rr * a.sk.t, g, kc, c);
      frag fv = dfrag<T, D>(vp + (int64_t)rr * a.sv.t, g, kc);
      if (row >= a.Tk) { fk = frag{}; fv = frag{}; }
      kf[ks][kc] = fk;
      vf[ks][kc] = fv;
    }
  }
  // FQ: wave w computes the dQ tile's d-block dtq = w % DT for its NQW
  // query sub-tiles qsq .. qsq + NQW - 1 (D = 64: all four), over the
  // block's keys.  A operands: dS rows from the dS^T tile; B operands: K
  // from the KS tile (rows past Tk read as zeros), both by transposed reads
  // (ltfrag), so the key order of the two agrees.
  constexpr int NQW = FQ ? DT : 1;
  const int dtq = wid % DT, qsq = (wid / DT) * DT;
  float* __restrict__ dqp = a.dq + b * a.sdq.b + h * a.sdq.h;
  const LaneOffs<T, BQ> lsq(n, g);
  // dQ[qt + 16 (qsq + i) + 4g + r][16 dtq + n] += scale * (dS K) from the
  // dS^T tile of query tile qt
  auto dq_phase = [&](const int qt) {
    if constexpr (FQ) {
      f32x4 acc[NQW];
#pragma unroll
      for (int i = 0; i < NQW; ++i) acc[i] = zero4();
#pragma unroll
      for (int s = 0; s < BKV / 32; ++s) {
        const frag kb = ltfrag<T, D>(KS, s, lo.t(dtq));
#pragma unroll
        for (int i = 0; i < NQW; ++i) acc[i] = MF::mma(ltfrag<T, BQ>(S0, s, lsq.t(qsq + i)), kb, acc[i]);
      }
#pragma unroll
      for (int i = 0; i < NQW; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qi = qt + 16 * (qsq + i) + 4 * g + r;
          if (qi < a.Tq) unsafeAtomicAdd(dqp + (int64_t)qi * a.sdq.t + 16 * dtq + n, acc[i][r] * a.scale);
        }
    }
  };
  // FQ: a key block that runs past Tk masks those keys in every tile (their
  // P would be exp(-lse), unbounded, and dS enters dQ)
  const bool rag = FQ && k0 + BKV > a.Tk;
  // one query tile; P = buffer parity (for direct loads the loop below is
  // unrolled by two so that P is a compile-time constant)
  // `open`: the tile is known to be fully visible to every wave of the
  // block (no skip, no mask), so the body has no branch around its MFMAs
  // and the accumulators stay in place (a branch there makes the compiler
  // copy all 64 of them per tile)
  auto step = [&](auto par, const int it, auto open) {
    constexpr bool OPEN = decltype(open)::value;
    const int P = int(par) % NBUF;
    const int PN = (P + 1) % NBUF;
    const int qt = qstart + it * BQ;
    LT* __restrict__ Qb = P ? Q1 : Q0;
    LT* __restrict__ Db = P ? D1 : D0;
    float* __restrict__ lse_b = P ? L1 : L0;
    float* __restrict__ del_b = P ? E1 : E0;
    if constexpr (LY::DIRECT) {
      wait_dma();
    } else {
      if constexpr (NBUF == 1) __syncthreads();
      qreg.put(Qb, LD, tid);
      dreg.put(Db, LD, tid);
    }
    if (tid < BQ) {
      const bool ok = qt + tid < a.Tq;
      lse_b[tid] = ok ? -lse_r * kLog2e : -INFINITY;
      del_b[tid] = ok ? -del_r : 0.f;
    }
    __syncthreads();
    if (it + 1 < ntile) fetch(qt + BQ, PN ? Q1 : Q0, PN ? D1 : D0);
    // FQ: every wave has finished the previous tile's dQ reads of S0 (barrier above)
    LT* __restrict__ Sb = S0;

    // wave-level causal skip: every key of the wave is after every query of the tile
    if (!OPEN && a.causal && kw0 > qt + BQ - 1 + off) {
      if constexpr (FQ) {
        // this wave's dS^T rows are zero
#pragma unroll
        for (int ks = 0; ks < NK; ++ks)
#pragma unroll
          for (int qs = 0; qs < BQ / 16; ++qs)
            *reinterpret_cast<uint2*>(Sb + LS::at(NK * 16 * wid + 16 * ks + n, 16 * qs + 4 * g)) = make_uint2(0u, 0u);
        __syncthreads();  // every wave passes one such barrier per tile
        dq_phase(qt);
      }
      return;
    }
    const bool need_mask = !OPEN && ((a.causal && (kw0 + NK * 16 - 1 > qt + off)) || rag);
    // dropout keep bytes of this lane's keys for queries qt + 16qs + 4g + r,
    // packed one query quad per word
    uint32_t kwd[BQ / 16][NK];
    if constexpr (DROP) {
#pragma unroll
      for (int qs = 0; qs < BQ / 16; ++qs)
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) {
          const int kj = min(kw0 + 16 * ks + n, a.Tk - 1);
          uint32_t w = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int qi = min(qt + 16 * qs + 4 * g + r, a.Tq - 1);
            w |= (uint32_t)(a.keep[((int64_t)bh * a.Tq + qi) * a.kld + kj] != 0) << (8 * r);
          }
          kwd[qs][ks] = w;
        }
    }
    auto tile = [&](auto masked) {
    constexpr bool MASKED = decltype(masked)::value;

    // The 64-query tile is walked in groups of GQ 16-query sub-tiles, one
    // group per dV/dK MFMA k-step (bf16: 32 queries; fp32: 16 queries = 4
    // steps).  Every LDS fragment is read once and feeds all NK key
    // sub-blocks of the wave; only one group's P / dS is live at a time.
    constexpr int GQ = MF::KI >= 16 ? MF::KI / 16 : 1;
    constexpr int NG = 4 / GQ;
    constexpr int SPG = NS / NG;
#pragma unroll
    for (int gq = 0; gq < NG; ++gq) {
      f32x4 p[NK][GQ], ds[NK][GQ];
#pragma unroll
      for (int j = 0; j < GQ; ++j) {
        const int qs = gq * GQ + j;
        frag qa[KC], da[KC];
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          qa[kc] = lfrag<T, D>(Qb + 16 * qs * LD + lo.d(kc));
          da[kc] = lfrag<T, D>(Db + 16 * qs * LD + lo.d(kc));
        }
        const f32x4 nlse = *reinterpret_cast<const f32x4*>(lse_b + 16 * qs + 4 * g);
        const f32x4 ndel = *reinterpret_cast<const f32x4*>(del_b + 16 * qs + 4 * g);
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) {
          f32x4 sv = nlse, dpv = ndel;
#pragma unroll
          for (int kc = 0; kc < KC; ++kc) {
            sv = MF::mma(qa[kc], kf[ks][kc], sv);
            dpv = MF::mma(da[kc], vf[ks][kc], dpv);
          }
          // key kj is hidden from query qt + ql iff r < kj - qt - off - 16qs - 4g
          const int hid = kw0 + 16 * ks + n - qt - off - 16 * qs - 4 * g;
          const bool kout = FQ && kw0 + 16 * ks + n >= a.Tk;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float pv = __builtin_amdgcn_exp2f(sv[r]);
            if (MASKED && need_mask && ((a.causal && r < hid) || kout)) pv = 0.f;
            if constexpr (DROP) {
              // dV takes the kept P; dS = P (z dP' - delta) with z = keep*kscale
              // and dP' = dO V^T (the product with the kept P); the MFMA gave
              // dpv = dP' - delta and ndel = -delta
              const float z = zf(kwd[qs][ks], r, a.kscale);
              p[ks][j][r] = pv * z;
              ds[ks][j][r] = pv * (z * (dpv[r] - ndel[r]) + ndel[r]);
            } else {
              p[ks][j][r] = pv;
              ds[ks][j][r] = pv * dpv[r];
            }
          }
        }
      }
#pragma unroll
      for (int ls = 0; ls < SPG; ++ls) {
        const int st = gq * SPG + ls;
        frag pb[NK], db[NK];
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) {
          pb[ks] = pfrag<T, GQ>(p[ks], ls);
          db[ks] = pfrag<T, GQ>(ds[ks], ls);
          if constexpr (FQ) {
            // dS^T row (key) NK*16 wid + 16 ks + n, queries 16 qs + 4g + 0..3
            // for the group's two sub-tiles qs = 2 gq, 2 gq + 1
            static_assert(!FQ || (GQ == 2 && SPG == 1), "one k-step per query group");
            const uint4 u = __builtin_bit_cast(uint4, db[ks]);
            const int row = NK * 16 * wid + 16 * ks + n;
            *reinterpret_cast<uint2*>(Sb + LS::at(row, 32 * gq + 4 * g)) = make_uint2(u.x, u.y);
            *reinterpret_cast<uint2*>(Sb + LS::at(row, 32 * gq + 16 + 4 * g)) = make_uint2(u.z, u.w);
          }
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const frag dof = ltfrag<T, D>(Db, st, lo.t(dt));
          const frag qf2 = ltfrag<T, D>(Qb, st, lo.t(dt));
#pragma unroll
          for (int ks = 0; ks < NK; ++ks) {
            dva[ks][dt] = MF::mma(dof, pb[ks], dva[ks][dt]);
            dka[ks][dt] = MF::mma(qf2, db[ks], dka[ks][dt]);
          }
        }
      }
    }
      };
    if constexpr (OPEN) {
      tile(std::false_type{});
    } else {
#if MTX_DKDV_SPLIT
      if (need_mask) tile(std::true_type{});
      else tile(std::false_type{});
#else
      tile(std::true_type{});
#endif
    }
    if constexpr (FQ) {
      __syncthreads();  // the tile's dS^T is complete
      dq_phase(qt);
    }
  };
  // Tiles from query qfull on see every key of the block: the first tiles
  // (at most BKV / BQ + 1 of them, rounded up to an even count for the
  // buffer parity) take the general body, the rest the open one.
  int itA = 0;
  if (a.causal) {
    const int qfull = k0 + BKV - 1 - off;
    itA = qfull > qstart ? (qfull - qstart + BQ - 1) / BQ : 0;
    itA = min(ntile, (itA + 1) & ~1);
  }
  if (rag) itA = ntile;
  if constexpr (LY::DIRECT) {
    for (int it = 0; it < itA; it += 2) {
      step(std::integral_constant<int, 0>{}, it, std::false_type{});
      if (it + 1 < itA) step(std::integral_constant<int, 1>{}, it + 1, std::false_type{});
    }
    for (int it = itA; it < ntile; it += 2) {
      step(std::integral_constant<int, 0>{}, it, std::true_type{});
      if (it + 1 < ntile) step(std::integral_constant<int, 1>{}, it + 1, std::true_type{});
    }
  } else {
    for (int it = 0; it < ntile; ++it) {
      if (it < itA) step(it & 1, it, std::false_type{});
      else step(it & 1, it, std::true_type{});
    }
  }

  float* __restrict__ dkp = a.dk + b * a.sdk.b + h * a.sdk.h;
  float* __restrict__ dvp = a.dv + b * a.sdv.b + h * a.sdv.h;
  const bool accf = a.accumulate != 0;
  if constexpr (GSTAGE) {
    // A store instruction straight from the accumulators writes 64 bytes of
    // each of 16 rows, so every 128-byte line reached memory in two
    // non-temporal pieces (1.41x the gradient bytes written).  The wave's
    // NK*16 rows go through LDS instead (the 16-byte chunks of row r
    // XOR-permuted by r mod D/4, so that at D = 64 neither the staging writes
    // nor the row reads meet in a bank) and each instruction writes
    // 64 / (D/4) whole rows of D floats.
    static_assert(D % 4 == 0 && 64 % (D / 4) == 0, "whole rows per wave store");
    constexpr int LPR = D / 4;           // lanes per row (16-byte chunks per row)
    constexpr int RPI = 64 / LPR;        // rows per store instruction
    constexpr int NR = NK * 16;          // the wave's rows
    float* __restrict__ ge = GE + wid * NR * D;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float* __restrict__ dst = t == 0 ? dkp : dvp;
      const int64_t st = t == 0 ? a.sdk.t : a.sdv.t;
      __syncthreads();  // (t = 1) every lane's reads of the dK rows are done
#pragma unroll
      for (int ks = 0; ks < NK; ++ks)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          *reinterpret_cast<f32x4*>(ge + (16 * ks + n) * D + 4 * ((4 * dt + g) ^ ((16 * ks + n) % LPR))) =
              t == 0 ? dka[ks][dt] * a.scale : dva[ks][dt];
      __syncthreads();
      const int rl = lane / LPR, c = lane % LPR;
#pragma unroll
      for (int r0 = 0; r0 < NR; r0 += RPI) {
        const int r = r0 + rl, kj = kw0 + r;
        if (kj < a.Tk)
          store_grad4(dst + (int64_t)kj * st + 4 * c, *reinterpret_cast<const f32x4*>(ge + r * D + 4 * (c ^ (r % LPR))),
                      accf);
      }
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
      const int kj = kw0 + 16 * ks + n;
      if (kj < a.Tk) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          store_grad4(dkp + (int64_t)kj * a.sdk.t + 16 * dt + 4 * g, dka[ks][dt] * a.scale, accf);
          store_grad4(dvp + (int64_t)kj * a.sdv.t + 16 * dt + 4 * g, dva[ks][dt], accf);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// backward, pass 2: dQ (query-outer, transposed products like the forward)
// ---------------------------------------------------------------------------
// FD: also computes delta[i] = sum_d dO[i,d] O[i,d] for its rows (from the
// same fragments it loads anyway) and writes it for the dK/dV pass.
template <typename T, int D, int NQ, bool FD, bool DROP>
__global__ __launch_bounds__(kThreads, (sizeof(T) == 2 && D <= 64) ? MTX_DQ_WAVES : (((D == 128 && sizeof(T) == 4) || (is_x3<T>() && D == 64 && MTX_X3_DQ_WAVES1)) ? 1 : 2))
void attn_dq_kernel(const BwdArgs a) {
  using MF = Mfma<T>;
  using frag = typename MF::frag;
  using DM = DMap<T, D>;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int KC = DM::KC;
  constexpr int DT = D / 16;
  constexpr int BQ = kWaves * NQ * 16;
  constexpr int BK = 64;
  constexpr int NS = BK / MF::KI;
  using LY = Lay<T, D>;
  constexpr int LD = LY::LD;
  constexpr int RSZ = BK * LD;
  using G = typename GEl<T>::type;   // element type in global memory
  using LT = typename LEl<T>::type;  // element type of the LDS tiles
  constexpr int NPLN = planes<T>();
  constexpr int NBUF = is_x3<T>() ? 1 : (sizeof(T) == 4 && D <= 64 && MTX_F32_NBUF1) ? 1 : (2 * RSZ * (int)sizeof(T) * 2 <= 80 * 1024 ? 2 : 1);
  static_assert(!LY::DIRECT || NBUF == 2, "direct tile loads need two buffers");
  // separate arrays per buffer, picked with compile-time parities (see the
  // forward kernel)
  __shared__ __attribute__((aligned(16))) LT K0[RSZ * NPLN], V0[RSZ * NPLN];
  __shared__ __attribute__((aligned(16))) LT K1[NBUF == 2 ? RSZ * NPLN : 1], V1[NBUF == 2 ? RSZ * NPLN : 1];

  const int BH = a.B * a.H;
  const int nqb = (a.Tq + BQ - 1) / BQ;
  int qb, bh;
  map_block(blockIdx.x, nqb, BH, a.causal != 0, qb, bh);
  const int b = bh / a.H, h = bh % a.H;
  const G* __restrict__ qp = static_cast<const G*>(a.q) + b * a.sq.b + h * a.sq.h;
  const G* __restrict__ kp = static_cast<const G*>(a.k) + b * a.sk.b + h * a.sk.h;
  const G* __restrict__ vp = static_cast<const G*>(a.v) + b * a.sv.b + h * a.sv.h;
  const G* __restrict__ dop = static_cast<const G*>(a.dout) + b * a.sdo.b + h * a.sdo.h;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int q0 = qb * BQ;
  const int qw0 = q0 + wid * NQ * 16;
  const int off = a.Tk - a.Tq;
  const float c = a.scale * kLog2e;

  // Q pre-multiplied by c = scale*log2(e); the S and dP MFMAs start from
  // -lse*log2(e) and -delta, so they yield log2(P) and dP - delta directly
  frag qf[NQ][KC], df[NQ][KC];
  f32x4 nlse[NQ], ndel[NQ];
#pragma unroll
  for (int qs = 0; qs < NQ; ++qs) {
    const int row = qw0 + 16 * qs + n;
    const bool ok = row < a.Tq;
    const int rr = ok ? row : a.Tq - 1;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      frag fq = dfrag_scaled<T, D>(qp + (int64_t)rr * a.sq.t, g, kc, c);
      frag fd = dfrag<T, D>(dop + (int64_t)rr * a.sdo.t, g, kc);
      if (!ok) { fq = frag{}; fd = frag{}; }
      qf[qs][kc] = fq;
      df[qs][kc] = fd;
    }
    const float nl = ok ? -a.lse[(int64_t)bh * a.Tq + row] * kLog2e : -INFINITY;
    float dl;
    if constexpr (FD) {
      // this lane's quarter of the row, then the sum over the 4 lanes of the row
      const G* __restrict__ orow = static_cast<const G*>(a.o) + b * a.so.b + h * a.so.h + (int64_t)rr * a.so.t;
      dl = 0.f;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if constexpr (is_x3<T>()) {
          // delta from the fp32 values (dO reloaded: its fragments are split)
          float ov[8], dv[8];
          load8<D>(orow, g, kc, ov);
          load8<D>(dop + (int64_t)rr * a.sdo.t, g, kc, dv);
#pragma unroll
          for (int e = 0; e < 8; ++e) dl = fmaf(ov[e], dv[e], dl);
        } else if constexpr (sizeof(T) == 4) {
          const frag fo = dfrag<T, D>(orow, g, kc);
          dl = fmaf(fo, df[qs][kc], dl);
        } else {
          const frag fo = dfrag<T, D>(orow, g, kc);
#pragma unroll
          for (int e = 0; e < 8; ++e) dl = fmaf((float)fo[e], (float)df[qs][kc][e], dl);
        }
      }
      dl = sum4l(dl);
      if (ok && g == 0) a.delta[(int64_t)bh * a.Tq + row] = dl;
    } else {
      dl = ok ? a.delta[(int64_t)bh * a.Tq + row] : 0.f;
    }
    const float nd = ok ? -dl : 0.f;
    nlse[qs] = f32x4{nl, nl, nl, nl};
    ndel[qs] = f32x4{nd, nd, nd, nd};
  }

  f32x4 acc[NQ][DT];
#pragma unroll
  for (int qs = 0; qs < NQ; ++qs)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[qs][dt] = zero4();

  const int kend = a.causal ? min(a.Tk, q0 + BQ + off) : a.Tk;
  const int ntile = (kend + BK - 1) / BK;
  const LaneOffs<T, D> lo(n, g);
  TileDma<T, BK, D> kdma, vdma;  // bf16: direct global -> LDS
  typename TileRegsSel<T, BK, D>::type kreg, vreg;  // fp32: through registers
  if constexpr (LY::DIRECT) {
    kdma.init(kp, a.sk.t, a.Tk, wid, lane);
    vdma.init(vp, a.sv.t, a.Tk, wid, lane);
    if (ntile > 0) {
      kdma.issue(0, K0, wid);
      vdma.issue(0, V0, wid);
    }
  } else if (ntile > 0) {
    kreg.fetch(kp, a.sk.t, 0, a.Tk, tid);
    vreg.fetch(vp, a.sv.t, 0, a.Tk, tid);
  }
  // one key tile; P = buffer parity (for direct loads the loop below is
  // unrolled by two so that P is a compile-time constant)
  // `open`: every key of the tile is visible to every query of the block
  // (no skip, no mask), so the body has no branch around its MFMAs and the
  // accumulators stay in place
  auto step = [&](auto par, const int it, auto open) {
    constexpr bool OPEN = decltype(open)::value;
    const int P = int(par) % NBUF;  // a constant for the unrolled (direct-load) loop
    const int PN = (P + 1) % NBUF;
    const int kb = it * BK;
    LT* __restrict__ Kb = P ? K1 : K0;
    LT* __restrict__ Vb = P ? V1 : V0;
    if constexpr (LY::DIRECT) {
      wait_dma();
    } else {
      if constexpr (NBUF == 1) __syncthreads();
      kreg.put(Kb, LD, tid);
      vreg.put(Vb, LD, tid);
    }
    __syncthreads();
    if (it + 1 < ntile) {
      if constexpr (LY::DIRECT) {
        kdma.issue(kb + BK, PN ? K1 : K0, wid);
        vdma.issue(kb + BK, PN ? V1 : V0, wid);
      } else {
        kreg.fetch(kp, a.sk.t, kb + BK, a.Tk, tid);
        vreg.fetch(vp, a.sv.t, kb + BK, a.Tk, tid);
      }
    }

    if (!OPEN && a.causal && kb > qw0 + NQ * 16 - 1 + off) return;
    const bool need_mask = !OPEN && ((kb + BK > a.Tk) || (a.causal && kb + BK - 1 > qw0 + off));
    // dropout keep bytes of this lane's query, keys kb + 16kt + 4g + 0..3
    uint32_t kwd[NQ][4];
    if constexpr (DROP) {
#pragma unroll
      for (int qs = 0; qs < NQ; ++qs) {
        const int64_t ro = ((int64_t)bh * a.Tq + min(qw0 + 16 * qs + n, a.Tq - 1)) * a.kld;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kwd[qs][kt] = keep4(a.keep, ro, kb + 16 * kt + 4 * g, a.kld);
      }
    }
    auto tile = [&](auto masked) {
    constexpr bool MASKED = decltype(masked)::value;

    // two 32-key halves: dS of a half, then its dQ products (only one
    // half's dS is live)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
    f32x4 ds[NQ][2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int kt = 2 * hf + kk;
      frag kfr[KC], vfr[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        kfr[kc] = lfrag<T, D>(Kb + 16 * kt * LD + lo.d(kc));
        vfr[kc] = lfrag<T, D>(Vb + 16 * kt * LD + lo.d(kc));
      }
#pragma unroll
      for (int qs = 0; qs < NQ; ++qs) {
        f32x4 sv = nlse[qs], dpv = ndel[qs];
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
          sv = MF::mma(kfr[kc], qf[qs][kc], sv);
          dpv = MF::mma(vfr[kc], df[qs][kc], dpv);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float pv = __builtin_amdgcn_exp2f(sv[r]);
          if constexpr (MASKED) {
            // key kb + 16kt + 4g + r is visible iff r <= lim
            int lim = a.Tk - 1 - kb - 16 * kt - 4 * g;
            if (a.causal) lim = min(lim, qw0 + 16 * qs + n + off - kb - 16 * kt - 4 * g);
            if (r > lim) pv = 0.f;
          }
          if constexpr (DROP) {
            // dS = P (z dP' - delta), dpv = dP' - delta (see the dK/dV pass)
            const float z = zf(kwd[qs][kt], r, a.kscale);
            ds[qs][kk][r] = pv * (z * (dpv[r] - ndel[qs][r]) + ndel[qs][r]);
          } else {
            ds[qs][kk][r] = pv * dpv[r];
          }
        }
      }
    }

#pragma unroll
    for (int st = hf * NS / 2; st < (hf + 1) * NS / 2; ++st) {
      frag db[NQ];
#pragma unroll
      for (int qs = 0; qs < NQ; ++qs) db[qs] = pfrag<T, 2>(ds[qs], st - hf * NS / 2);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const frag kt_f = ltfrag<T, D>(Kb, st, lo.t(dt));
#pragma unroll
        for (int qs = 0; qs < NQ; ++qs) acc[qs][dt] = MF::mma(kt_f, db[qs], acc[qs][dt]);
      }
    }
    }
      };
    if constexpr (OPEN) {
      tile(std::false_type{});
    } else {
      if (need_mask) tile(std::true_type{});
      else tile(std::false_type{});
    }
  };
  // Key tiles below kopen are visible to every query of the block: those
  // (an even count, for the buffer parity) take the open body, the rest
  // (the diagonal and the ragged end) the general one.
  const int kopen = a.causal ? min(a.Tk, q0 + off + 1) : a.Tk;
  const int itB = min(ntile, kopen / BK) & ~1;
  if constexpr (LY::DIRECT) {
    for (int it = 0; it < itB; it += 2) {
      step(std::integral_constant<int, 0>{}, it, std::true_type{});
      step(std::integral_constant<int, 1>{}, it + 1, std::true_type{});
    }
    for (int it = itB; it < ntile; it += 2) {
      step(std::integral_constant<int, 0>{}, it, std::false_type{});
      if (it + 1 < ntile) step(std::integral_constant<int, 1>{}, it + 1, std::false_type{});
    }
  } else {
    for (int it = 0; it < ntile; ++it) {
      if (it < itB) step(it & 1, it, std::true_type{});
      else step(it & 1, it, std::false_type{});
    }
  }

  float* __restrict__ dqp = a.dq + b * a.sdq.b + h * a.sdq.h;
  const bool accf = a.accumulate != 0;
  if constexpr (BF && D == 64 && kWaves == 4 && NBUF == 2) {
    // A store instruction straight from the accumulators writes 64 bytes of
    // each of 16 rows, so every 128-byte line reached memory in two
    // non-temporal pieces.  Each wave stages its NQ*16 rows of dQ in one of
    // the four K/V tile buffers, free after the loop (rows of 64 floats, the
    // 16-byte chunks of row r XOR-permuted by r % 16, so that neither the
    // staging writes nor the row reads meet in a bank), and each store
    // instruction writes 4 whole rows.
    constexpr int NR = NQ * 16;
    static_assert((int)sizeof(K0) >= NR * D * (int)sizeof(float), "a wave's rows fit one tile buffer");
    __syncthreads();  // every wave's reads of the K/V tiles are done
    float* __restrict__ ge = reinterpret_cast<float*>(wid == 0 ? K0 : wid == 1 ? V0 : wid == 2 ? K1 : V1);
#pragma unroll
    for (int qs = 0; qs < NQ; ++qs) {
      const int r = 16 * qs + n;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(ge + r * D + 4 * ((4 * dt + g) ^ (r & 15))) = acc[qs][dt] * a.scale;
    }
    __syncthreads();
    const int rl = lane >> 4, c = lane & 15;
#pragma unroll
    for (int r0 = 0; r0 < NR; r0 += 4) {
      const int r = r0 + rl, qi = qw0 + r;
      if (qi < a.Tq)
        store_grad4(dqp + (int64_t)qi * a.sdq.t + 4 * c, *reinterpret_cast<const f32x4*>(ge + r * D + 4 * (c ^ (r & 15))),
                    accf);
    }
  } else {
#pragma unroll
    for (int qs = 0; qs < NQ; ++qs) {
      const int qi = qw0 + 16 * qs + n;
      if (qi < a.Tq) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          store_grad4(dqp + (int64_t)qi * a.sdq.t + 16 * dt + 4 * g, acc[qs][dt] * a.scale, accf);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// tile parameters per dtype
// NQ: 16-query sub-tiles per wave (forward, dQ); NK: 16-key sub-tiles per
// wave (dK/dV).  Larger values reuse each LDS fragment for more MFMAs; they
// are capped where the accumulators would no longer fit 2 waves per SIMD.
// Compile-time tuning knobs (bf16, D <= 64), overridable with -D for sweeps.
#ifndef MTX_FWD_NQ_BF16
#define MTX_FWD_NQ_BF16 2
#endif
#ifndef MTX_DQ_NQ_BF16
#define MTX_DQ_NQ_BF16 2
#endif
#ifndef MTX_DKDV_NK_BF16
#define MTX_DKDV_NK_BF16 2
#endif
template <typename T, int D> struct Cfg;
template <int D> struct Cfg<float, D> { static constexpr int NQ = 1, NK = 1, NQF = 1; };
template <int D> struct Cfg<f32x3_t, D> {
  static constexpr int NQ = D == 64 ? MTX_X3_NQ : 1, NK = D == 64 ? MTX_X3_NK : 1, NQF = 1;
};
template <int D> struct Cfg<bf16_t, D> {
  static constexpr int NQ = D <= 64 ? MTX_DQ_NQ_BF16 : 1;
  static constexpr int NQF = D <= 64 ? MTX_FWD_NQ_BF16 : 2;
  static constexpr int NK = D <= 64 ? MTX_DKDV_NK_BF16 : 1;
};

int check_bhtd(const char* name, const void* p, const int64_t* s, int esize) {
  MTX_CHECK_ARG(p != nullptr, "%s: null pointer", name);
  MTX_CHECK_ARG(s != nullptr, "%s: null strides", name);
  MTX_CHECK_ARG(s[3] == 1, "%s: the d stride must be 1 (got %lld)", name, (long long)s[3]);
  const int vec = 16 / esize;
  for (int i = 0; i < 3; ++i)
    MTX_CHECK_ARG(s[i] >= 0 && s[i] % vec == 0,
                  "%s: stride[%d]=%lld must be a non-negative multiple of %d elements", name, i,
                  (long long)s[i], vec);
  MTX_CHECK_ARG(((uintptr_t)p & 15u) == 0, "%s: pointer must be 16-byte aligned", name);
  // tile loads use 32-bit offsets from a tile's first row
  MTX_CHECK_SHAPE(s[2] < (1 << 24), "%s: the t stride (%lld elements) must be < 2^24", name, (long long)s[2]);
  return MTX_OK;
}

// bf16 tiles load through a buffer resource spanning one (b,h) slice's rows:
// rows * t_stride * 2 bytes must stay below 2^31
int check_slice_bytes(const char* name, const int64_t* s, int rows, int esize) {
  if (esize != 2) return MTX_OK;
  MTX_CHECK_SHAPE((int64_t)rows * s[2] * esize < ((int64_t)1 << 31),
                  "%s: %d rows x t stride %lld x 2 bytes must be < 2^31 (bf16 tile loads)", name, rows,
                  (long long)s[2]);
  return MTX_OK;
}

int check_dims(int dtype, int B, int H, int Tq, int Tk, int D, int causal) {
  if (dtype != MTX_F32 && dtype != MTX_BF16) return fail(MTX_ERR_DTYPE, "unsupported dtype %d", dtype);
  MTX_CHECK_SHAPE(B >= 1 && H >= 1 && Tq >= 1 && Tk >= 1, "B,H,Tq,Tk must be >= 1 (got %d,%d,%d,%d)",
                  B, H, Tq, Tk);
  MTX_CHECK_SHAPE(D == 16 || D == 32 || D == 64 || D == 128, "head dim D=%d not in {16,32,64,128}", D);
  MTX_CHECK_SHAPE(!causal || Tq <= Tk, "causal attention needs Tq <= Tk (got %d > %d)", Tq, Tk);
  MTX_CHECK_SHAPE((int64_t)B * H <= (1 << 24) && Tq <= (1 << 24) && Tk <= (1 << 24), "shape too large");
  return MTX_OK;
}

Str3 s3(const int64_t* s) { return Str3{s[0], s[1], s[2]}; }

template <typename T, int D>
int launch_fwd(const FwdArgs& a, hipStream_t st) {
  constexpr int NQ = Cfg<T, D>::NQF;
  constexpr int BQ = kWaves * NQ * 16;
  const int grid = cdiv(a.Tq, BQ) * a.B * a.H;
  if (a.keep)
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, NQ, true>), dim3(grid), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, NQ, false>), dim3(grid), dim3(kThreads), 0, st, a);
  MTX_LAUNCHED();
  return MTX_OK;
}

// Backward structure for the full gradient (MTX_ATTN_BWD_ALL): the
// deterministic two passes (the default), or for bf16 with D <= 64 the
// one-pass kernel (mtx_attn_set_bwd_mode MTX_ATTN_BWD_ONEPASS).  Measured at
// B=8, H=16, T=2048, D=64: one-pass 26 us (delta, dq zeroed) + 485 us
// (key-outer with dQ atomics; 314 us with the atomics taken out) against
// 103 us (dQ pass) + 141 us (dK/dV pass): 570 MB of fp32 atomic adds into dq
// cost more than the dQ pass's recomputed S and dP.
std::atomic<int> g_bwd_mode{MTX_ATTN_BWD_TWOPASS};

template <typename T, int D>
constexpr bool has_onepass() {
  return sizeof(T) == 2 && D <= 64 && Cfg<T, D>::NK == 2 && dkdv_waves<T>() == 4;
}

// One-pass phases: MTX_ATTN_BWD_ONEPASS | DELTA runs the preparation kernel
// (delta; dq zeroed unless accumulating), ONEPASS | DQ | DKDV the one-pass
// kernel (dK, dV written, dQ added into dq).
template <typename T, int D>
int launch_onepass(const BwdArgs& a, int phases, hipStream_t st) {
  if constexpr (has_onepass<T, D>()) {
    constexpr int NK = Cfg<T, D>::NK;
    if (phases & MTX_ATTN_BWD_DELTA) {
      const int64_t lanes = (int64_t)a.B * a.H * a.Tq * 4;
      hipLaunchKernelGGL((attn_prep_kernel<T, D>), dim3((unsigned)((lanes + kThreads - 1) / kThreads)),
                         dim3(kThreads), 0, st, a);
      MTX_LAUNCHED();
    }
    if (phases & (MTX_ATTN_BWD_DQ | MTX_ATTN_BWD_DKDV)) {
      constexpr int NWV = dkdv_waves<T>();
      const int gk = cdiv(a.Tk, NWV * NK * 16) * a.B * a.H;
      hipLaunchKernelGGL((attn_dkdv_kernel<T, D, NK, false, true>), dim3(gk), dim3(64 * NWV), 0, st, a);
      MTX_LAUNCHED();
    }
    return MTX_OK;
  } else {
    return fail(MTX_ERR_SHAPE, "the one-pass backward needs bf16 inputs and D <= 64");
  }
}

// Phase order: delta, dQ, dK/dV.  DELTA together with DQ runs as one
// kernel (the dQ pass computes delta for its rows and stores it), which the
// dK/dV pass then reads.
template <typename T, int D>
int launch_bwd(const BwdArgs& a, int phases, hipStream_t st) {
  constexpr int NQ = Cfg<T, D>::NQ, NK = Cfg<T, D>::NK;
  if (phases & MTX_ATTN_BWD_ONEPASS) return launch_onepass<T, D>(a, phases, st);
  if constexpr (has_onepass<T, D>()) {
    if (phases == MTX_ATTN_BWD_ALL && !a.keep && g_bwd_mode.load(std::memory_order_relaxed) == MTX_ATTN_BWD_ONEPASS)
      return launch_onepass<T, D>(a, phases, st);
  }
  const bool fuse = (phases & MTX_ATTN_BWD_DELTA) && (phases & MTX_ATTN_BWD_DQ);
  if ((phases & MTX_ATTN_BWD_DELTA) && !fuse) {
    const int64_t rows = (int64_t)a.B * a.H * a.Tq;
    hipLaunchKernelGGL((attn_delta_kernel<typename GEl<T>::type, D>), dim3((unsigned)((rows + kThreads - 1) / kThreads)),
                       dim3(kThreads), 0, st, a);
    MTX_LAUNCHED();
  }
  if (phases & MTX_ATTN_BWD_DQ) {
    const int gq = cdiv(a.Tq, kWaves * NQ * 16) * a.B * a.H;
    if (a.keep) {
      if (fuse)
        hipLaunchKernelGGL((attn_dq_kernel<T, D, NQ, true, true>), dim3(gq), dim3(kThreads), 0, st, a);
      else
        hipLaunchKernelGGL((attn_dq_kernel<T, D, NQ, false, true>), dim3(gq), dim3(kThreads), 0, st, a);
    } else {
      if (fuse)
        hipLaunchKernelGGL((attn_dq_kernel<T, D, NQ, true, false>), dim3(gq), dim3(kThreads), 0, st, a);
      else
        hipLaunchKernelGGL((attn_dq_kernel<T, D, NQ, false, false>), dim3(gq), dim3(kThreads), 0, st, a);
    }
    MTX_LAUNCHED();
  }
  if (phases & MTX_ATTN_BWD_DKDV) {
    constexpr int NWV = dkdv_waves<T>();
    const int gk = cdiv(a.Tk, NWV * NK * 16) * a.B * a.H;
    if (a.keep)
      hipLaunchKernelGGL((attn_dkdv_kernel<T, D, NK, true>), dim3(gk), dim3(64 * NWV), 0, st, a);
    else
      hipLaunchKernelGGL((attn_dkdv_kernel<T, D, NK, false>), dim3(gk), dim3(64 * NWV), 0, st, a);
    MTX_LAUNCHED();
  }
  return MTX_OK;
}

template <typename T>
int dispatch_fwd(int D, const FwdArgs& a, hipStream_t st) {
  switch (D) {
    case 16: return launch_fwd<T, 16>(a, st);
    case 32: return launch_fwd<T, 32>(a, st);
    case 64: return launch_fwd<T, 64>(a, st);
    default: return launch_fwd<T, 128>(a, st);
  }
}

template <typename T>
int dispatch_bwd(int D, const BwdArgs& a, int phases, hipStream_t st) {
  switch (D) {
    case 16: return launch_bwd<T, 16>(a, phases, st);
    case 32: return launch_bwd<T, 32>(a, phases, st);
    case 64: return launch_bwd<T, 64>(a, phases, st);
    default: return launch_bwd<T, 128>(a, phases, st);
  }
}

// fp32 attention with 64-wide heads runs on the bf16 matrix cores
// (T = f32x3_t) unless mtx_attn_set_mode chose the fp32 MFMA kernels.
// Smaller heads stay on fp32 MFMA: at D = 16, T = 32 (the C0 model's
// attention, latency bound) the split's staging work made the training step
// 17% slower.
std::atomic<int> g_attn_mode{MTX_GEMM_BF16X3};

bool use_x3(int dtype, int D) {
  return dtype == MTX_F32 && D == 64 && g_attn_mode.load(std::memory_order_relaxed) == MTX_GEMM_BF16X3;
}

int dispatch_fwd_x3(const FwdArgs& a, hipStream_t st) { return launch_fwd<f32x3_t, 64>(a, st); }

int dispatch_bwd_x3(const BwdArgs& a, int phases, hipStream_t st) { return launch_bwd<f32x3_t, 64>(a, phases, st); }

}  // namespace
}  // namespace mtx

using namespace mtx;

extern "C" int mtx_attn_set_mode(int mode) {
  MTX_CHECK_ARG(mode == MTX_GEMM_FP32 || mode == MTX_GEMM_BF16X3,
                "attention mode %d must be MTX_GEMM_FP32 (0) or MTX_GEMM_BF16X3 (1)", mode);
  g_attn_mode.store(mode);
  return MTX_OK;
}

extern "C" int mtx_attn_get_mode(void) { return g_attn_mode.load(); }

extern "C" int mtx_attn_set_bwd_mode(int mode) {
  MTX_CHECK_ARG(mode == MTX_ATTN_BWD_ONEPASS || mode == MTX_ATTN_BWD_TWOPASS,
                "bwd mode must be MTX_ATTN_BWD_ONEPASS (%d) or MTX_ATTN_BWD_TWOPASS (%d), got %d",
                MTX_ATTN_BWD_ONEPASS, MTX_ATTN_BWD_TWOPASS, mode);
  g_bwd_mode.store(mode);
  return MTX_OK;
}

extern "C" int mtx_attn_get_bwd_mode(void) { return g_bwd_mode.load(); }

namespace {
int check_keep(const uint8_t* keep, int64_t keep_ld, float keep_scale, int Tk) {
  if (!keep) return MTX_OK;
  MTX_CHECK_ARG(((uintptr_t)keep & 3u) == 0, "keep: pointer must be 4-byte aligned");
  MTX_CHECK_ARG(keep_ld >= Tk && keep_ld % 4 == 0,
                "keep_ld=%lld must be >= Tk=%d and a multiple of 4", (long long)keep_ld, Tk);
  MTX_CHECK_ARG(std::isfinite(keep_scale) && keep_scale > 0.f, "keep_scale must be finite and > 0");
  return MTX_OK;
}

int attn_fwd_impl(int dtype, int B, int H, int Tq, int Tk, int D,
                  const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                  const void* v, const int64_t* v_strides, void* o, const int64_t* o_strides,
                  float* lse, float scale, int causal, const uint8_t* keep, int64_t keep_ld,
                  float keep_scale, void* stream) {
  int rc = check_dims(dtype, B, H, Tq, Tk, D, causal);
  if (rc) return rc;
  const int es = dtype == MTX_F32 ? 4 : 2;
  if ((rc = check_bhtd("q", q, q_strides, es))) return rc;
  if ((rc = check_bhtd("k", k, k_strides, es))) return rc;
  if ((rc = check_bhtd("v", v, v_strides, es))) return rc;
  if ((rc = check_bhtd("o", o, o_strides, es))) return rc;
  if ((rc = check_slice_bytes("k", k_strides, Tk, es))) return rc;
  if ((rc = check_slice_bytes("v", v_strides, Tk, es))) return rc;
  if ((rc = check_keep(keep, keep_ld, keep_scale, Tk))) return rc;
  MTX_CHECK_ARG(lse != nullptr, "lse: null pointer");
  MTX_CHECK_ARG(std::isfinite(scale) && scale > 0.f, "scale must be finite and > 0");
  FwdArgs a{q, s3(q_strides), k, s3(k_strides), v, s3(v_strides), o, s3(o_strides),
            lse, B, H, Tq, Tk, scale, causal ? 1 : 0, keep, keep_ld, keep_scale};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_x3(dtype, D)) return dispatch_fwd_x3(a, st);
  return dtype == MTX_F32 ? dispatch_fwd<float>(D, a, st) : dispatch_fwd<bf16_t>(D, a, st);
}
}  // namespace

extern "C" int mtx_attn_fwd(int dtype, int B, int H, int Tq, int Tk, int D,
                            const void* q, const int64_t* q_strides,
                            const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides,
                            void* o, const int64_t* o_strides,
                            float* lse, float scale, int causal, void* stream) {
  return attn_fwd_impl(dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides, v, v_strides, o, o_strides,
                       lse, scale, causal, nullptr, 0, 1.f, stream);
}

extern "C" int mtx_attn_fwd_dropout(int dtype, int B, int H, int Tq, int Tk, int D,
                                    const void* q, const int64_t* q_strides,
                                    const void* k, const int64_t* k_strides,
                                    const void* v, const int64_t* v_strides,
                                    void* o, const int64_t* o_strides,
                                    float* lse, float scale, int causal,
                                    const uint8_t* keep, int64_t keep_ld, float keep_scale,
                                    void* stream) {
  MTX_CHECK_ARG(keep != nullptr, "keep: null pointer");
  return attn_fwd_impl(dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides, v, v_strides, o, o_strides,
                       lse, scale, causal, keep, keep_ld, keep_scale, stream);
}

// ---------------------------------------------------------------------------
// Backward without allocation: the delta rows live in a file-scope device
// array instead of a caller-supplied workspace.  Each GPU holds its own copy
// (MTX_ATTN_SCRATCH_BYTES, kept until the process ends); host code reaches it
// only through the address hipGetSymbolAddress returns for the current device,
// looked up once per device (at mtx_device_init, or on the first call).  Calls
// that overlap on one GPU share the array and race.  Nothing in it needs to
// start at zero: the dQ pass writes every delta row before the dK/dV pass
// reads it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[MTX_ATTN_SCRATCH_BYTES / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_rc[kMaxDevices];
}  // namespace

namespace mtx {
// Address of the current device's scratch array (looked up on first use).
int attn_scratch(void** out) {
  int dev = -1;
  MTX_HIP(hipGetDevice(&dev));
  MTX_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = p;
  });
  if (g_scratch_rc[dev] != hipSuccess)
    return fail(MTX_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(g_scratch_rc[dev]));
  *out = g_scratch_ptr[dev];
  return MTX_OK;
}
}  // namespace mtx

extern "C" size_t mtx_attn_bwd_workspace_bytes(int B, int H, int Tq) {
  if (B < 1 || H < 1 || Tq < 1) return 0;
  return (size_t)B * H * Tq * sizeof(float);
}

namespace {
int attn_bwd_impl(int phases, int dtype, int B, int H, int Tq, int Tk, int D,
                            const void* q, const int64_t* q_strides,
                            const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides,
                            const void* o, const int64_t* o_strides,
                            const void* dout, const int64_t* do_strides,
                            const float* lse,
                            float* dq, const int64_t* dq_strides,
                            float* dk, const int64_t* dk_strides,
                            float* dv, const int64_t* dv_strides,
                            void* workspace, size_t workspace_bytes,
                            float scale, int causal, int accumulate,
                            const uint8_t* keep, int64_t keep_ld, float keep_scale, void* stream,
                            bool use_scratch = false) {
  MTX_CHECK_ARG(phases > 0 && (phases & ~(MTX_ATTN_BWD_ALL | MTX_ATTN_BWD_ONEPASS)) == 0 &&
                    (phases & MTX_ATTN_BWD_ALL) != 0,
                "bad phase mask %d", phases);
  if (phases & MTX_ATTN_BWD_ONEPASS) {
    MTX_CHECK_SHAPE(dtype == MTX_BF16 && D <= 64 && keep == nullptr,
                    "MTX_ATTN_BWD_ONEPASS phases need bf16 inputs, D <= 64 and no dropout");
    MTX_CHECK_ARG((phases & MTX_ATTN_BWD_DQ) == 0 || (phases & MTX_ATTN_BWD_DKDV) != 0,
                  "the one-pass kernel computes dQ and dK/dV together (phases DQ | DKDV)");
  }
  int rc = check_dims(dtype, B, H, Tq, Tk, D, causal);
  if (rc) return rc;
  const int es = dtype == MTX_F32 ? 4 : 2;
  if ((rc = check_bhtd("q", q, q_strides, es))) return rc;
  if ((rc = check_bhtd("k", k, k_strides, es))) return rc;
  if ((rc = check_bhtd("v", v, v_strides, es))) return rc;
  if ((rc = check_bhtd("o", o, o_strides, es))) return rc;
  if ((rc = check_bhtd("dout", dout, do_strides, es))) return rc;
  if ((rc = check_bhtd("dq", dq, dq_strides, 4))) return rc;
  if ((rc = check_bhtd("dk", dk, dk_strides, 4))) return rc;
  if ((rc = check_bhtd("dv", dv, dv_strides, 4))) return rc;
  if ((rc = check_slice_bytes("q", q_strides, Tq, es))) return rc;
  if ((rc = check_slice_bytes("k", k_strides, Tk, es))) return rc;
  if ((rc = check_slice_bytes("v", v_strides, Tk, es))) return rc;
  if ((rc = check_slice_bytes("dout", do_strides, Tq, es))) return rc;
  MTX_CHECK_ARG(lse != nullptr, "lse: null pointer");
  if (!use_scratch) {
    MTX_CHECK_ARG(workspace != nullptr, "workspace: null pointer");
    MTX_CHECK_ARG(workspace_bytes >= mtx_attn_bwd_workspace_bytes(B, H, Tq),
                  "workspace too small: %zu < %zu bytes", workspace_bytes,
                  mtx_attn_bwd_workspace_bytes(B, H, Tq));
  }
  MTX_CHECK_ARG(std::isfinite(scale) && scale > 0.f, "scale must be finite and > 0");
  if ((rc = check_keep(keep, keep_ld, keep_scale, Tk))) return rc;
  if (use_scratch && (rc = attn_scratch(&workspace))) return rc;  // after validation: no HIP call before it
  BwdArgs a{q, s3(q_strides), k, s3(k_strides), v, s3(v_strides), o, s3(o_strides),
            dout, s3(do_strides), lse, static_cast<float*>(workspace),
            dq, s3(dq_strides), dk, s3(dk_strides), dv, s3(dv_strides),
            B, H, Tq, Tk, scale, causal ? 1 : 0, accumulate ? 1 : 0, keep, keep_ld, keep_scale};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_x3(dtype, D)) return dispatch_bwd_x3(a, phases, st);
  return dtype == MTX_F32 ? dispatch_bwd<float>(D, a, phases, st)
                          : dispatch_bwd<bf16_t>(D, a, phases, st);
}

}  // namespace

extern "C" int mtx_attn_bwd_phase(int phases, int dtype, int B, int H, int Tq, int Tk, int D,
                            const void* q, const int64_t* q_strides,
                            const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides,
                            const void* o, const int64_t* o_strides,
                            const void* dout, const int64_t* do_strides,
                            const float* lse,
                            float* dq, const int64_t* dq_strides,
                            float* dk, const int64_t* dk_strides,
                            float* dv, const int64_t* dv_strides,
                            void* workspace, size_t workspace_bytes,
                            float scale, int causal, int accumulate, void* stream) {
  return attn_bwd_impl(phases, dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides, v, v_strides, o,
                       o_strides, dout, do_strides, lse, dq, dq_strides, dk, dk_strides, dv, dv_strides,
                       workspace, workspace_bytes, scale, causal, accumulate, nullptr, 0, 1.f, stream);
}

extern "C" int mtx_attn_bwd_dropout(int dtype, int B, int H, int Tq, int Tk, int D,
                                    const void* q, const int64_t* q_strides,
                                    const void* k, const int64_t* k_strides,
                                    const void* v, const int64_t* v_strides,
                                    const void* o, const int64_t* o_strides,
                                    const void* dout, const int64_t* do_strides,
                                    const float* lse,
                                    float* dq, const int64_t* dq_strides,
                                    float* dk, const int64_t* dk_strides,
                                    float* dv, const int64_t* dv_strides,
                                    void* workspace, size_t workspace_bytes,
                                    float scale, int causal, int accumulate,
                                    const uint8_t* keep, int64_t keep_ld, float keep_scale,
                                    void* stream) {
  MTX_CHECK_ARG(keep != nullptr, "keep: null pointer");
  return attn_bwd_impl(MTX_ATTN_BWD_ALL, dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides, v,
                       v_strides, o, o_strides, dout, do_strides, lse, dq, dq_strides, dk, dk_strides,
                       dv, dv_strides, workspace, workspace_bytes, scale, causal, accumulate, keep,
                       keep_ld, keep_scale, stream);
}

extern "C" int mtx_attn_bwd_noalloc(int dtype, int B, int H, int Tq, int Tk, int D,
                                    const void* q, const int64_t* q_strides,
                                    const void* k, const int64_t* k_strides,
                                    const void* v, const int64_t* v_strides,
                                    const void* o, const int64_t* o_strides,
                                    const void* dout, const int64_t* do_strides,
                                    const float* lse,
                                    float* dq, const int64_t* dq_strides,
                                    float* dk, const int64_t* dk_strides,
                                    float* dv, const int64_t* dv_strides,
                                    float scale, int causal, int accumulate, void* stream) {
  MTX_CHECK_SHAPE(B >= 1 && H >= 1 && Tq >= 1, "B,H,Tq must be >= 1 (got %d,%d,%d)", B, H, Tq);
  const size_t need = mtx_attn_bwd_workspace_bytes(B, H, Tq);
  MTX_CHECK_SHAPE(need <= (size_t)MTX_ATTN_SCRATCH_BYTES,
                  "mtx_attn_bwd_noalloc: B*H*Tq = %lld rows need %zu bytes of delta, more than the "
                  "library's fixed %zu-byte scratch (B*H*Tq <= %zu); use mtx_attn_bwd with a workspace",
                  (long long)B * H * Tq, need, (size_t)MTX_ATTN_SCRATCH_BYTES,
                  (size_t)MTX_ATTN_SCRATCH_BYTES / sizeof(float));
  return attn_bwd_impl(MTX_ATTN_BWD_ALL, dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides, v,
                       v_strides, o, o_strides, dout, do_strides, lse, dq, dq_strides, dk, dk_strides,
                       dv, dv_strides, nullptr, (size_t)MTX_ATTN_SCRATCH_BYTES, scale, causal, accumulate,
                       nullptr, 0, 1.f, stream, /*use_scratch=*/true);
}

extern "C" int mtx_attn_bwd(int dtype, int B, int H, int Tq, int Tk, int D,
                            const void* q, const int64_t* q_strides,
                            const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides,
                            const void* o, const int64_t* o_strides,
                            const void* dout, const int64_t* do_strides,
                            const float* lse,
                            float* dq, const int64_t* dq_strides,
                            float* dk, const int64_t* dk_strides,
                            float* dv, const int64_t* dv_strides,
                            void* workspace, size_t workspace_bytes,
                            float scale, int causal, int accumulate, void* stream) {
  return mtx_attn_bwd_phase(MTX_ATTN_BWD_ALL, dtype, B, H, Tq, Tk, D, q, q_strides, k, k_strides,
                            v, v_strides, o, o_strides, dout, do_strides, lse, dq, dq_strides,
                            dk, dk_strides, dv, dv_strides, workspace, workspace_bytes, scale,
                            causal, accumulate, stream);
}
