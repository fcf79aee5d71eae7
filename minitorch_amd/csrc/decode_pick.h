// Greedy pick helpers shared by the decode kernels (gfx950): the top two
// values of a row with np.argmax's order, and the pick's per-row
// bookkeeping.
#pragma once
#include "mtx_common.h"

namespace mtx {

// ---- greedy pick: first maximum per row and top-2 margin ----
// np.argmax's order: a NaN ranks above every number (the first NaN is the
// pick), otherwise the first maximum; a row of -Inf picks its first index.
// i1 == n_cols marks "nothing seen yet" (a lane with no columns).
struct Top2 {
  float m1, m2;
  int i1;
};

// a ranks above b
__device__ __forceinline__ bool above(float a, float b) { return a > b || (a != a && b == b); }
__device__ __forceinline__ float top(float a, float b) { return above(b, a) ? b : a; }

// column c (scanned in increasing order) with value v
__device__ __forceinline__ void scan(Top2& t, float v, int c, int ncols) {
  if (t.i1 == ncols || above(v, t.m1)) {
    if (t.i1 != ncols) t.m2 = t.m1;
    t.m1 = v;
    t.i1 = c;
  } else {
    t.m2 = top(t.m2, v);
  }
}

__device__ __forceinline__ Top2 merge(Top2 x, Top2 y, int ncols) {
  if (y.i1 == ncols) return x;
  if (x.i1 == ncols) return y;
  Top2 r;
  const bool xa = above(x.m1, y.m1), ya = above(y.m1, x.m1);
  const bool xw = xa || (!ya && x.i1 < y.i1);  // ties: the lower index
  r.m1 = xw ? x.m1 : y.m1;
  r.i1 = xw ? x.i1 : y.i1;
  r.m2 = xw ? top(x.m2, y.m1) : top(y.m2, x.m1);
  return r;
}

__device__ __forceinline__ Top2 reduce_top2(Top2 t, int ncols) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    Top2 o;
    o.m1 = __shfl_xor(t.m1, m, 64);
    o.m2 = __shfl_xor(t.m2, m, 64);
    o.i1 = __shfl_xor(t.i1, m, 64);
    t = merge(t, o, ncols);
  }
  return t;
}

// The pick's bookkeeping for one row (lane 0): the next input id, the id
// and margin records, the row's length and (row 0) the position id.
__device__ __forceinline__ void pick_record(int row, int rows, const Top2& t, int64_t* __restrict__ cur,
                                            int64_t* __restrict__ ids, int Tmax, float* __restrict__ margins,
                                            int t_base, int nm, int* __restrict__ lengths,
                                            int64_t* __restrict__ pos) {
  const int L = lengths[row];
  cur[row] = t.i1;
  if (L >= 0 && L < Tmax) ids[(int64_t)L * rows + row] = t.i1;
  const int s = L - t_base;
  if (margins != nullptr && s >= 0 && s < nm) margins[(int64_t)s * rows + row] = t.m1 - t.m2;
  lengths[row] = L + 1;
  if (row == 0 && pos != nullptr) pos[0] += 1;
}

}  // namespace mtx
