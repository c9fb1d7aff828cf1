// fp32 sums in the order of torch's CPU reduction kernel, for kernels whose results must equal
// the reference's fp32 reductions bit for bit.
#pragma once
#include "common.h"

namespace {

// ---------------------------------------------------------------------------------------------
// fp32 sums in the order of torch's CPU reduction kernel (aten/src/ATen/native/cpu/SumKernel.cpp,
// cascade_sum), which computes the reference's Gini sums and head means (routing.py:99-101):
//   * cascade: one accumulator chain over n elements, pushed up a 4-level cascade every 2^p
//     elements (p = max(4, ceil(log2 n) / 4)) and folded at the end (multi_row_sum);
//   * row_sum: 4 interleaved cascades over n / 4 groups, the tail added to the first, then the
//     four folded in order;
//   * inner_sum: a contiguous run of n >= 8 is summed as 8 lanes (lane l = row_sum of elements
//     l, l + 8, ...), then the scalar tail and the 8 lanes are added one by one to 0; n < 8 uses
//     row_sum directly.
// One thread evaluates these sequentially with round-to-nearest adds (no contraction or
// reassociation), so the result is bit-identical to the reference's fp32 value.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int tc_ceil_log2(int n) {
  if (n <= 2) return 1;
  return 32 - __clz((unsigned)(n - 1));
}

template <typename Load>
__device__ float tc_cascade(const Load& x, int start, int stride, int n) {
  const int power = max(4, tc_ceil_log2(n) / 4);
  const int step = 1 << power, mask = step - 1;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int i = 0;
  while (i + step <= n) {
    for (int j = 0; j < step; ++j, ++i) acc[0] = wa_add_rn(acc[0], x(start + i * stride));
    for (int j = 1; j < 4; ++j) {
      acc[j] = wa_add_rn(acc[j], acc[j - 1]);
      acc[j - 1] = 0.f;
      if ((i & (mask << (j * power))) != 0) break;
    }
  }
  for (; i < n; ++i) acc[0] = wa_add_rn(acc[0], x(start + i * stride));
  for (int j = 1; j < 4; ++j) acc[0] = wa_add_rn(acc[0], acc[j]);
  return acc[0];
}

template <typename Load>
__device__ float tc_row_sum(const Load& x, int start, int stride, int n) {
  const int groups = n / 4;
  float part[4];
  for (int k = 0; k < 4; ++k) part[k] = tc_cascade(x, start + k * stride, 4 * stride, groups);
  for (int i = groups * 4; i < n; ++i) part[0] = wa_add_rn(part[0], x(start + i * stride));
  for (int k = 1; k < 4; ++k) part[0] = wa_add_rn(part[0], part[k]);
  return part[0];
}

template <typename Load>
__device__ float tc_inner_sum(const Load& x, int start, int n) {
  constexpr int L = 8;
  if (n < L) return tc_row_sum(x, start, 1, n);
  const int nv = n / L;
  float fin = 0.f;
  for (int k = nv * L; k < n; ++k) fin = wa_add_rn(fin, x(start + k));
  for (int l = 0; l < L; ++l) fin = wa_add_rn(fin, tc_row_sum(x, start + l, L, nv));
  return fin;
}

// tc_inner_sum with its 32 independent cascades (lane l's cascade k runs over elements
// start + l + 8 k + 32 i) on threads base .. base + 31 of the workgroup, then the same folds in the
// same order on thread `base`: the same fp32 value. Every thread of the workgroup calls it (it
// holds a barrier); `chain` is 32 floats of LDS; the result is valid on thread `base`.
template <typename Load>
__device__ float tc_inner_sum_wg(const Load& x, int start, int n, float* chain, int base = 0) {
  constexpr int L = 8;
  const int t = (int)threadIdx.x - base;
  if (n < L) return t == 0 ? tc_row_sum(x, start, 1, n) : 0.f;
  const int nv = n / L, groups = nv / 4;
  if (t >= 0 && t < 32) chain[t] = tc_cascade(x, start + (t % 8) + 8 * (t / 8), 4 * L, groups);
  __syncthreads();
  float fin = 0.f;
  if (t == 0) {
    for (int k = nv * L; k < n; ++k) fin = wa_add_rn(fin, x(start + k));
    for (int l = 0; l < L; ++l) {
      float part = chain[l];
      for (int i = groups * 4; i < nv; ++i) part = wa_add_rn(part, x(start + l + i * L));
      for (int k = 1; k < 4; ++k) part = wa_add_rn(part, chain[l + 8 * k]);
      fin = wa_add_rn(fin, part);
    }
  }
  return fin;
}

}  // namespace
