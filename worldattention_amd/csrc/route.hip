// Block routing kernels: block mean pooling, block attention map + stable descending sort +
// selection (Gini cumulative mass or per-head top-k), and mask -> index compaction.
//
// Reference semantics: wan/modules/hsa/routing.py:45-118 and block_sparse_triton.py:20-57.
#include <algorithm>

#include "common.h"
#include "tile.h"
#include "torch_order.h"

namespace {

// ---------------------------------------------------------------------------------------------
// Block mean pooling (routing.py:45-61). One workgroup per (block, head, batch); every thread
// reads 16 bytes per token row and accumulates in fp32; the row slots are summed through LDS.
// ---------------------------------------------------------------------------------------------
struct PoolParams {
  const void* x; int64_t sb, st, sh; int dtype;
  int L, H, D, Bs, N;
  const int32_t* heads;
  float* out;
  int emulate;
  int nh;  // head slots (heads listed, or H)
  int blk0, n_out, sums;  // first block of the launch, blocks of the output, write sums
};

// Several pooling jobs (e.g. the query and key tensors of one call) in one launch: job j takes
// workgroups [start[j], start[j + 1]) of a 1-D grid.
constexpr int POOL_MAX_JOBS = 4;
struct PoolJobs {
  PoolParams job[POOL_MAX_JOBS];
  int64_t start[POOL_MAX_JOBS + 1];
  int n;
};

// The block mean of routing.py:45-61 from the fp32 sum of the block's `real` tokens of a tensor of
// L tokens: with L a multiple of the block size, the mean in the input dtype (a bf16 input rounds
// it), otherwise the sum in the input dtype divided by the real count in fp32.
__device__ __forceinline__ float block_mean_from_sum(float s, int L, int Bs, int real, bool bf) {
  if (L % Bs == 0) {
    const float m = s / (float)Bs;
    return bf ? wa_bf16_round(m) : m;
  }
  return (bf ? wa_bf16_round(s) : s) / (float)real;
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256) pool_kernel(PoolJobs pj) {
  extern __shared__ float red[];  // [rows_per_pass][D + 4]
  const int64_t id = blockIdx.x;
  int j = 0;
  while (j + 1 < pj.n && id >= pj.start[j + 1]) ++j;
  const PoolParams& p = pj.job[j];
  // consecutive workgroups take the heads of one token block: they read neighbouring chunks of the
  // same token rows
  const int64_t local = id - pj.start[j];
  const int hs = (int)(local % p.nh), blk = p.blk0 + (int)((local / p.nh) % p.N),
            b = (int)(local / ((int64_t)p.nh * p.N));
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tpr = p.D / VEC;             // threads per token row
  const int rpp = 256 / tpr;             // token rows per pass
  const int tid = threadIdx.x;
  const int slot = tid / tpr, col = (tid % tpr) * VEC;
  const int real = max(0, min(p.Bs, p.L - blk * p.Bs));
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
  if (slot < rpp) {
    const T* base = (const T*)p.x + (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)blk * p.Bs * p.st + col;
    // rows slot, slot + rpp, ...: groups of POOL_BATCH loads issued together, then summed in order
    constexpr int POOL_BATCH = 8;
    for (int t0 = slot; t0 < real; t0 += POOL_BATCH * rpp) {
      T v[POOL_BATCH][VEC];
#pragma unroll
      for (int k = 0; k < POOL_BATCH; ++k) {
        const int t = t0 + k * rpp;
        const T* src = base + (int64_t)(t < real ? t : 0) * p.st;
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[k][i] = src[i];
      }
#pragma unroll
      for (int k = 0; k < POOL_BATCH; ++k) {
        if (t0 + k * rpp < real) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] += (float)v[k][i];
        }
      }
    }
    // row stride D + 4 floats: the rows a wave stores land in different banks
#pragma unroll
    for (int i = 0; i < VEC; ++i) red[slot * (p.D + 4) + col + i] = acc[i];
  }
  __syncthreads();
  for (int d = tid; d < p.D; d += 256) {
    float s = 0.f;
    for (int r = 0; r < rpp; ++r) s += red[r * (p.D + 4) + d];
    float m = s;
    if (!p.sums) m = block_mean_from_sum(s, p.L, p.Bs, real, p.emulate && p.dtype == WA_BF16);
    p.out[(((int64_t)b * p.H + h) * p.n_out + blk) * p.D + d] = m;
  }
}

// ---------------------------------------------------------------------------------------------
// Routing of one row (batch, head, query block): probabilities, bitonic sort of
// (probability desc, block id asc) keys in LDS, permutation + count (+ Gini inputs).
// ---------------------------------------------------------------------------------------------
struct RouteParams {
  const float* probs; const float* qp; const float* kp;
  int B, H, Nq, Nkv, D, NP, n_heads;
  int mode;
  float tau_min, tau_span, scale;
  const int32_t* head_k;
  const int32_t* heads;
  int32_t* index; int32_t* num; float* thresholds; uint8_t* mask; float* probs_out;
  float* ws_sorted; float* ws_gini;
  int32_t* clear; int64_t n_clear;
  int k_sum_len, Bs, k_sum_bf16;  // k_pooled holds block sums of k_sum_len tokens (0: means)
  int kp_blocks;                  // blocks per (batch, head) row of k_pooled (>= Nkv)
  float inv_bs;                   // 1 / Bs when Bs is a power of two (exact), else 0
  int k_sum_div;                  // k_sum_len % Bs == 0
};

// Pooled key element of block j: the stored mean, or the mean formed from the stored sum
// (block_mean_from_sum). Used by the loops that visit a key row element by element.
__device__ __forceinline__ float pooled_key(const RouteParams& p, float x, int j) {
  if (p.k_sum_len <= 0) return x;
  const int real = max(1, min(p.Bs, p.k_sum_len - j * p.Bs));
  return block_mean_from_sum(x, p.k_sum_len, p.Bs, real, p.k_sum_bf16 != 0);
}

// A whole key row held in registers, sums -> means. For a power-of-two block size a full block's
// division is a multiply by the exact reciprocal (the same correctly rounded result), so one branch
// per row picks the multiply for every block but a partial last one, which divides.
template <int NC>
__device__ __forceinline__ void pooled_key_row(const RouteParams& p, f32x4 (&kv)[NC], int j) {
  if (p.k_sum_len <= 0) return;
  const bool bf = p.k_sum_bf16 != 0;
  if (p.inv_bs != 0.f && (j < p.Nkv - 1 || p.k_sum_div)) {
    const bool pre = bf && !p.k_sum_div, post = bf && p.k_sum_div;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = pre ? wa_bf16_round(kv[c][e]) : kv[c][e];
        const float m = x * p.inv_bs;
        kv[c][e] = post ? wa_bf16_round(m) : m;
      }
    }
  } else {
    const float real = (float)max(1, min(p.Bs, p.k_sum_len - j * p.Bs));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < 4; ++e) kv[c][e] = (bf ? wa_bf16_round(kv[c][e]) : kv[c][e]) / real;
    }
  }
}

__device__ __forceinline__ float block_reduce_max(float v, float* scratch) {
  v = wa_wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  float r = scratch[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, scratch[i]);
  return r;
}

__device__ __forceinline__ double block_reduce_sum_d(double v, double* scratch) {
  v = wa_wave_sum_d(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += scratch[i];
  return r;
}

// Outputs the row kernels do not produce, written by one extra workgroup (the last x index of
// the grid, y = z = 0): num = 0 for the rows of heads outside the routed list, thresholds = 0
// for every head without a Gini threshold, and the caller's `clear` words. Returns true for every
// workgroup of that last x index.
__device__ bool clear_unrouted(const RouteParams& p) {
  if (blockIdx.x != gridDim.x - 1) return false;
  if (blockIdx.y | blockIdx.z) return true;
  auto routed = [&](int h) {
    if (!p.heads) return true;
    for (int s = 0; s < p.n_heads; ++s)
      if (p.heads[s] == h) return true;
    return false;
  };
  if (p.thresholds)
    for (int h = threadIdx.x; h < p.H; h += blockDim.x)
      if (p.mode != WA_ROUTE_GINI || !routed(h)) p.thresholds[h] = 0.f;
  if (p.heads)
    for (int64_t u = threadIdx.x; u < (int64_t)p.B * p.H * p.Nq; u += blockDim.x)
      if (!routed((int)((u / p.Nq) % p.H))) p.num[u] = 0;
  for (int64_t u = threadIdx.x; u < p.n_clear; u += blockDim.x) p.clear[u] = 0;
  return true;
}

// tc_head_sum with its contiguous inner sums spread over threads base .. base + 31
// (tc_inner_sum_wg); every thread calls it, the result is valid on thread `base`.
template <typename Load>
__device__ float tc_head_sum_wg(const Load& g, int B, int H, int Nq, int h, float* chain, int base) {
  if (H == 1) return tc_inner_sum_wg(g, 0, B * Nq, chain, base);
  if (Nq == 1) return (int)threadIdx.x == base ? tc_head_sum(g, B, H, Nq, h) : 0.f;
  float s = 0.f;
  for (int b = 0; b < B; ++b) {
    const float part = tc_inner_sum_wg(g, (b * H + h) * Nq, Nq, chain, base);
    if ((int)threadIdx.x == base) s = wa_add_rn(s, part);
    __syncthreads();  // the chain buffer is reused
  }
  return s;
}

// Sum over (batch, query block) of one head's row Ginis g[(b * H + h) * Nq + i], as torch sums
// a [B, H, Nq] tensor over dims (0, 2): with H == 1 the two dims merge into one contiguous run;
// with Nq == 1 it is an outer reduction over b of column h (columns in groups of 32 when H >= 8,
// of 4 when H < 8, take one cascade each; the other columns a row_sum); otherwise the per-batch
// inner sums over Nq are added in batch order.
template <typename Load>
__device__ float tc_head_sum(const Load& g, int B, int H, int Nq, int h) {
  if (H == 1) return tc_inner_sum(g, 0, B * Nq);
  if (Nq == 1) {
    const int grouped = H >= 8 ? H / 32 * 32 : H / 4 * 4;
    return h < grouped ? tc_cascade(g, h, H, B) : tc_row_sum(g, h, H, B);
  }
  float s = 0.f;
  for (int b = 0; b < B; ++b) s = wa_add_rn(s, tc_inner_sum(g, (b * H + h) * Nq, Nq));
  return s;
}

__device__ __forceinline__ float key_to_float(uint64_t key) {
  const uint32_t u = (uint32_t)(key >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

__global__ void __launch_bounds__(256) route_kernel(RouteParams p) {
  extern __shared__ uint64_t keys[];        // [NP]
  __shared__ float qrow[256];
  __shared__ double dscratch[8];
  __shared__ float fscratch[8];
  __shared__ float fscratch32[32];
  if (clear_unrouted(p)) return;
  const int i = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x;
  const int64_t row = ((int64_t)b * p.H + h) * p.Nq + i;
  const int N = p.Nkv;

  // 1. block attention probabilities of this row
  float* pr = (float*)keys;  // reuse the key buffer for the fp32 row (NP*8 bytes >= N*4)
  if (p.probs) {
    for (int j = tid; j < N; j += 256) pr[j] = p.probs[row * N + j];
    __syncthreads();
  } else {
    const float* qsrc = p.qp + row * p.D;
    for (int d = tid; d < p.D; d += 256) qrow[d] = qsrc[d];
    __syncthreads();
    // 8 threads per key row: thread tg of the group reads d = 32k + 4tg .. +3 (coalesced float4).
    const float* kbase = p.kp + ((int64_t)b * p.H + h) * (int64_t)p.kp_blocks * p.D;
    const int grp = tid >> 3, tg = tid & 7;
    const bool vec = (p.D & 31) == 0;
    auto finish = [&](float s, int j) {
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 4, 64);
      if (j < N && tg == 0) pr[j] = s * p.scale;
    };
    if (vec && p.D == 128) {
      // four key groups per pass, their 16 loads in flight together (rows past N re-read the last)
      constexpr int U = 4;
      for (int j0 = 0; j0 < N; j0 += 32 * U) {
        f32x4 kv[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float* kr = kbase + (int64_t)min(j0 + 32 * u + grp, N - 1) * 128;
#pragma unroll
          for (int c = 0; c < 4; ++c) kv[u][c] = *(const f32x4*)(kr + 32 * c + 4 * tg);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = j0 + 32 * u + grp;
          f32x4 kr4[4] = {kv[u][0], kv[u][1], kv[u][2], kv[u][3]};
          pooled_key_row(p, kr4, min(j, N - 1));
          float s = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int d = 32 * c + 4 * tg;
            s = fmaf(qrow[d], kr4[c][0], s);
            s = fmaf(qrow[d + 1], kr4[c][1], s);
            s = fmaf(qrow[d + 2], kr4[c][2], s);
            s = fmaf(qrow[d + 3], kr4[c][3], s);
          }
          finish(s, j);
        }
      }
    } else {
      for (int j0 = 0; j0 < N; j0 += 32) {
        const int j = j0 + grp;
        float s = 0.f;
        if (j < N) {
          const float* kr = kbase + (int64_t)j * p.D;
          if (vec) {
            for (int d = 4 * tg; d < p.D; d += 32) {
              f32x4 kv[1] = {*(const f32x4*)(kr + d)};
              pooled_key_row(p, kv, j);
              s = fmaf(qrow[d], kv[0][0], s);
              s = fmaf(qrow[d + 1], kv[0][1], s);
              s = fmaf(qrow[d + 2], kv[0][2], s);
              s = fmaf(qrow[d + 3], kv[0][3], s);
            }
          } else {
            for (int d = tg; d < p.D; d += 8) s = fmaf(qrow[d], pooled_key(p, kr[d], j), s);
          }
        }
        finish(s, j);
      }
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int j = tid; j < N; j += 256) mx = fmaxf(mx, pr[j]);
    mx = block_reduce_max(mx, fscratch);
    double se = 0.0;
    for (int j = tid; j < N; j += 256) {
      const float e = expf(pr[j] - mx);
      pr[j] = e;
      se += (double)e;
    }
    se = block_reduce_sum_d(se, dscratch);
    const float inv_sum = (float)(1.0 / se);
    for (int j = tid; j < N; j += 256) {
      const float pj = pr[j] * inv_sum;
      pr[j] = pj;
      if (p.probs_out) p.probs_out[row * N + j] = pj;
    }
    __syncthreads();
  }

  // 2. composite keys: (probability ascending-order bits) << 32 | ~block id; padding = 0.
  uint64_t mine[16];
  const int per = p.NP / 256 > 0 ? p.NP / 256 : 1;
  for (int e = 0; e < per; ++e) {
    const int j = tid + e * 256;
    uint64_t kv = 0;
    if (j < N) kv = ((uint64_t)wa_float_key(pr[j]) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j);
    mine[e] = kv;
  }
  __syncthreads();
  for (int e = 0; e < per; ++e) {
    const int j = tid + e * 256;
    if (j < p.NP) keys[j] = mine[e];
  }
  __syncthreads();

  // 3. bitonic sort, descending
  for (int size = 2; size <= p.NP; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = tid; t < p.NP / 2; t += 256) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const uint64_t a = keys[lo], c = keys[hi];
        if ((a < c) == desc) {
          keys[lo] = c;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }

  // 4. permutation, count, gini inputs
  int32_t* idx_row = p.index + row * N;
  for (int m = tid; m < N; m += 256) idx_row[m] = (int32_t)(0xFFFFFFFFu - (uint32_t)keys[m]);
  if (p.mode == WA_ROUTE_TOPK) {
    const int kk = p.head_k ? p.head_k[h] : N;
    const int n = max(0, min(kk, N));
    if (tid == 0) p.num[row] = n;
    if (p.mask) {
      uint8_t* mrow = p.mask + row * N;
      for (int m = tid; m < N; m += 256) mrow[(int32_t)(0xFFFFFFFFu - (uint32_t)keys[m])] = m < n ? 1 : 0;
    }
  } else {
    // Gini terms (N + 1 - 2 m) p_(m), each rounded to fp32 as the reference's product tensor is,
    // then their sum in the reference's fp32 order, divided by N in fp32
    float terms[16];
    for (int e = 0; e < per; ++e) {
      const int m = tid + e * 256;
      terms[e] = 0.f;
      if (m < N) {
        const float pm = key_to_float(keys[m]);
        p.ws_sorted[row * N + m] = pm;
        terms[e] = wa_mul_rn((float)(N + 1 - 2 * (m + 1)), pm);
      }
    }
    __syncthreads();  // every key read: the buffer takes the terms
    float* tl = (float*)keys;
    for (int e = 0; e < per; ++e) {
      const int m = tid + e * 256;
      if (m < N) tl[m] = terms[e];
    }
    __syncthreads();
    const float s = tc_inner_sum_wg([&](int m) { return tl[m]; }, 0, N, fscratch32);
    if (tid == 0) p.ws_gini[row] = wa_div_rn(s, (float)N);
  }
}

// Top-k routing, R rows (query blocks i0 .. i0 + R - 1 of one head) per workgroup, rows of at most
// 512 blocks (R = 2: twice the workgroups in flight of R = 4, 14.8 -> 13.5 us at cfg 2; R = 1 is
// 16 us). Scores: thread t owns key j (= t, t + 256, ...) and forms its R rows' dot products from
// one pass over the key's pooled vector (the rows share the head's pooled keys; the pooled queries
// are broadcast from LDS). Then one wave per row: slot e*64 + lane lives in
// register e of the lane, so the softmax reduces over the wave and the bitonic network runs in
// registers (strides >= 64) and lane shuffles (strides < 64) without further barriers. The
// softmax takes the max, fp32 exponentials and a double row sum, then p = e * (1 / sum).
// The value of lane ^ stride (stride a power of two below 64, a constant after unrolling) by VALU
// lane moves: DPP quad permutes (1, 2), row shifts (4), a row rotate (8) and the gfx950 half-row
// and half-wave swaps (16, 32). Through ds_bpermute, each of the sort's dependent steps waited on
// the LDS crossbar: the sort took ~11,600 cycles of a ~27,000-cycle workgroup.
__device__ __forceinline__ uint32_t xor_lanes(uint32_t v, int stride, int lane) {
  switch (stride) {
    case 1: return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
    case 2: return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2, 3, 0, 1]
    case 4: {
      const uint32_t up = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0xF, false);  // row_shl:4 (lane + 4)
      const uint32_t dn = __builtin_amdgcn_update_dpp(v, v, 0x114, 0xF, 0xF, false);  // row_shr:4 (lane - 4)
      return (lane & 4) ? dn : up;
    }
    case 8: return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    case 16: {
      const auto sw = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // {odd rows <- lane - 16, even <- + 16}
      return (lane & 16) ? sw[0] : sw[1];
    }
    default: {
      const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // {upper half <- lane - 32, lower <- + 32}
      return (lane & 32) ? sw[0] : sw[1];
    }
  }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m, int lane) {
  const uint32_t lo = xor_lanes((uint32_t)v, m, lane);
  const uint32_t hi = xor_lanes((uint32_t)(v >> 32), m, lane);
  return ((uint64_t)hi << 32) | lo;
}

template <int KPL, int DK, int R, bool SUMS>
__global__ void __launch_bounds__(256) route_wave_kernel(RouteParams p) {
  constexpr int NP = 64 * KPL;
  // With the head dim known, the head's pooled keys are staged here (row j, 16-byte chunk c in slot
  // c ^ (j % (DK / 4)): a thread's row reads are then conflict-free across 16 lanes).
  __shared__ __attribute__((aligned(1024))) float k_sh[DK ? NP : 1][DK ? DK : 4];
  __shared__ __attribute__((aligned(16))) float q_sh[R][256];
  __shared__ float s_sh[R][NP];
  __shared__ __attribute__((aligned(16))) float last_sh[SUMS ? 256 : 4];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
  if (clear_unrouted(p)) return;
  const int i0 = blockIdx.x * R, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;  // uniform per workgroup
  const int N = p.Nkv, D = DK ? DK : p.D;
  const int64_t row0 = ((int64_t)b * p.H + h) * p.Nq;
  const float* kbase = p.kp + ((int64_t)b * p.H + h) * (int64_t)p.kp_blocks * D;

  // 1. scores of the four rows. With the head dim known at compile time (and N <= 256: one key
  // block per thread), this thread's pooled key row is loaded whole before the pooled queries are
  // staged, so both latencies overlap.
  // With cached sums and a power-of-two block size, a partial last block is the only row whose
  // means divide: the workgroup converts it once into LDS instead of one thread dividing D times.
  const bool last_in_lds = SUMS && p.inv_bs != 0.f && !p.k_sum_div;
  f32x4 kv[DK ? DK / 4 : 1];
  // The head's pooled key rows [0, N) go to LDS by direct-to-LDS loads, 1 KiB (RPI whole rows)
  // per wave instruction. Loading each thread's row into registers took ~11,000 cycles of a
  // ~27,000-cycle workgroup: every load instruction touched 64 rows 512 bytes apart.
  constexpr int CPR = DK ? DK / 4 : 1, RPI = 64 / CPR;
  if constexpr (DK != 0) {
    const int nins = (N + 4 * RPI - 1) / (4 * RPI);
    for (int i = 0; i < nins; ++i) {
      const int r0 = (i * 4 + w) * RPI, row = r0 + lane / CPR, slot = lane % CPR;
      const int rr = min(row, N - 1);  // rows past the head's keys repeat the last (never read)
      lds_dma16_global(kbase + (int64_t)rr * D + (slot ^ (row % CPR)) * 4, &k_sh[r0][0]);
    }
  }
  if constexpr (SUMS) {
    if (last_in_lds) {
      const float* kr = kbase + (int64_t)(N - 1) * D;
      const float real = (float)(p.k_sum_len - (N - 1) * p.Bs);
      for (int d = tid; d < D; d += 256) last_sh[d] = (p.k_sum_bf16 ? wa_bf16_round(kr[d]) : kr[d]) / real;
    }
  }
  for (int u = tid; u < R * D; u += 256) {
    const int r = u / D, d = u % D;
    q_sh[r][d] = i0 + r < p.Nq ? p.qp[(row0 + i0 + r) * D + d] : 0.f;
  }
  if constexpr (DK != 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's key rows landed
  __syncthreads();
  if constexpr (DK != 0) {
    // this thread's key row (as the pooled means: from cached sums the row is converted)
    const int jj = min(tid, N - 1);
#pragma unroll
    for (int c = 0; c < CPR; ++c) kv[c] = *(const f32x4*)(&k_sh[jj][(c ^ (jj % CPR)) * 4]);
    if constexpr (SUMS) {
      if (last_in_lds && jj == N - 1) {
#pragma unroll
        for (int c = 0; c < DK / 4; ++c) kv[c] = *(const f32x4*)(&last_sh[4 * c]);
      } else {
        pooled_key_row(p, kv, jj);
      }
    }
  }
  for (int j = tid; j < N; j += 256) {
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    if (DK) {
      // groups of four chunks: the fences keep the compiler from hoisting every LDS read of the
      // pooled queries ahead of the products (which would not fit in registers)
#pragma unroll
      for (int c0 = 0; c0 < DK / 4; c0 += 4) {
#pragma unroll
        for (int c = c0; c < c0 + 4; ++c) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const f32x4 qv = *(const f32x4*)(&q_sh[r][4 * c]);
            acc[r] = fmaf(qv[0], kv[c][0], acc[r]);
            acc[r] = fmaf(qv[1], kv[c][1], acc[r]);
            acc[r] = fmaf(qv[2], kv[c][2], acc[r]);
            acc[r] = fmaf(qv[3], kv[c][3], acc[r]);
          }
        }
        asm volatile("" ::: "memory");
      }
    } else {
      const float* kr = kbase + (int64_t)j * D;
      if ((D & 31) == 0) {
        for (int d0 = 0; d0 < D; d0 += 32) {
          f32x4 kc[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            kc[c] = *(const f32x4*)(kr + d0 + 4 * c);
          }
          if constexpr (SUMS) {
            if (last_in_lds && j == N - 1) {
#pragma unroll
              for (int c = 0; c < 8; ++c) kc[c] = *(const f32x4*)(&last_sh[d0 + 4 * c]);
            } else {
              pooled_key_row(p, kc, j);
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
              const f32x4 qv = *(const f32x4*)(&q_sh[r][d0 + 4 * c]);
              acc[r] = fmaf(qv[0], kc[c][0], acc[r]);
              acc[r] = fmaf(qv[1], kc[c][1], acc[r]);
              acc[r] = fmaf(qv[2], kc[c][2], acc[r]);
              acc[r] = fmaf(qv[3], kc[c][3], acc[r]);
            }
          }
        }
      } else {
        for (int d = 0; d < D; ++d) {
          const float kd = SUMS ? (last_in_lds && j == N - 1 ? last_sh[d] : pooled_key(p, kr[d], j)) : kr[d];
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] = fmaf(q_sh[r][d], kd, acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) s_sh[r][j] = acc[r] * p.scale;
  }
  __syncthreads();
  // With two rows per workgroup each row's softmax and sort run on two waves (half h of the row:
  // positions 128 h + 64 e + lane), so all four waves work; one row per wave took ~9,500 cycles
  // of sorting on one wave per SIMD. The halves meet through LDS for the softmax max and sum
  // (added in half order) and for the sort's one stride that crosses them (128, at size 256).
  constexpr bool SPLIT = R == 2 && KPL >= 2;
  constexpr int KW = SPLIT ? KPL / 2 : KPL;  // keys per lane of a wave
  __shared__ float red_mx[4];
  __shared__ double red_se[4];
  __shared__ uint64_t xk[SPLIT ? 4 : 1][SPLIT ? 64 * KW : 1];
  const int rw = SPLIT ? w >> 1 : w, hw = SPLIT ? (w & 1) : 0;
  const int i = i0 + rw;
  const bool active = rw < R && i < p.Nq;  // an inactive wave of a split row still meets the barriers
  if (!SPLIT && !active) return;
  const int64_t row = row0 + i;
  float* ss = s_sh[rw < R ? rw : 0];
  const int pos0 = hw * 64 * KW;  // first row position of this wave

  // 2. softmax over the row
  float sc[KW];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < KW; ++e) {
    const int j = pos0 + e * 64 + lane;
    sc[e] = j < N ? ss[j] : -INFINITY;
    mx = fmaxf(mx, sc[e]);
  }
  mx = wa_wave_max(mx);
  if constexpr (SPLIT) {
    if (lane == 0) red_mx[w] = mx;
    __syncthreads();
    mx = fmaxf(red_mx[w & ~1], red_mx[w | 1]);
  }
  double se = 0.0;
#pragma unroll
  for (int e = 0; e < KW; ++e) {
    const int j = pos0 + e * 64 + lane;
    sc[e] = j < N ? expf(sc[e] - mx) : 0.f;
    se += (double)sc[e];
  }
  se = wa_wave_sum_d(se);
  if constexpr (SPLIT) {
    if (lane == 0) red_se[w] = se;
    __syncthreads();
    se = red_se[w & ~1] + red_se[w | 1];
  }
  const float inv_sum = (float)(1.0 / se);

  // 3. composite keys (probability order bits, inverted block id), padding 0; bitonic, descending
  uint64_t key[KW];
#pragma unroll
  for (int e = 0; e < KW; ++e) {
    const int j = pos0 + e * 64 + lane;
    key[e] = j < N ? (((uint64_t)wa_float_key(sc[e] * inv_sum) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)j)) : 0ull;
  }
#pragma unroll
  for (int size = 2; size <= NP; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (SPLIT && stride == 64 * KW) {
        // the partner is the same slot of the row's other wave
#pragma unroll
        for (int e = 0; e < KW; ++e) xk[w][e * 64 + lane] = key[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < KW; ++e) {
          const uint64_t other = xk[w ^ 1][e * 64 + lane];
          const bool lower = hw == 0;
          const bool desc = ((pos0 + e * 64 + lane) & size) == 0;
          const bool keep = (key[e] > other) == (lower == desc);
          key[e] = keep ? key[e] : other;
        }
      } else if (stride >= 64) {
        const int es = stride >> 6;
#pragma unroll
        for (int e = 0; e < KW; ++e) {
          const int pe = e ^ es;
          if (pe > e) {
            const bool desc = ((pos0 + e * 64 + lane) & size) == 0;
            const uint64_t a = key[e], c = key[pe];
            if ((a < c) == desc) {
              key[e] = c;
              key[pe] = a;
            }
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < KW; ++e) {
          const uint64_t other = shfl_xor_u64(key[e], stride, lane);
          const bool lower = (lane & stride) == 0;
          const bool desc = ((pos0 + e * 64 + lane) & size) == 0;
          // keep the larger key where this lane takes the maximum, else the smaller (one compare,
          // one select; keys are distinct but for the equal zero padding)
          const bool keep = (key[e] > other) == (lower == desc);
          key[e] = keep ? key[e] : other;
        }
      }
    }
  }
  if (!active) return;

  // 4. permutation and count
  int32_t* idx_row = p.index + row * N;
  const int kk = p.head_k ? p.head_k[h] : N;
  const int n = max(0, min(kk, N));
#pragma unroll
  for (int e = 0; e < KW; ++e) {
    const int m = pos0 + e * 64 + lane;
    if (m < N) {
      const int32_t id = (int32_t)(0xFFFFFFFFu - (uint32_t)key[e]);
      idx_row[m] = id;
      if (p.mask) p.mask[row * N + id] = m < n ? 1 : 0;
    }
  }
  if (lane == 0 && hw == 0) p.num[row] = n;
}

// Gini second pass: per-head threshold (mean of the head's row Ginis), then the count of sorted
// slots whose exclusive prefix is below it. The prefix is the reference's: a sequential double
// running sum rounded to fp32, minus the slot's own weight in fp32 (routing.py:95-113). Two
// sequential chains run side by side, each on lane 0 of its own wave: the running sum (wave 0,
// which leaves every slot's exclusive prefix in LDS) and the head's mean Gini (wave 1); then all
// lanes compare the prefixes with the threshold and count.
constexpr int GINI_STAGE_MAX = 8192;  // row Ginis of a head staged in LDS up to this many

__global__ void __launch_bounds__(128) gini_count_kernel(RouteParams p) {
  // [N] sorted probabilities, then the exclusive prefixes; then (up to GINI_STAGE_MAX) this head's
  // row Ginis
  extern __shared__ float sp[];
  __shared__ float s_thr;
  __shared__ int s_cnt[2];
  __shared__ float s_chain[32];
  const int i = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row = ((int64_t)b * p.H + h) * p.Nq + i;
  const int N = p.Nkv;

  // the head's row Ginis g[(b H + h) Nq + i] to LDS in one round of loads (read inside the
  // sequential sum, each global load waited for the previous add), with the row's sorted weights
  const float* gw = p.ws_gini;
  const int BN = p.B * p.Nq;
  const bool staged = BN <= GINI_STAGE_MAX;
  float* sg = sp + N;
  if (staged)
    for (int u = tid; u < BN; u += 128) sg[u] = gw[((int64_t)(u / p.Nq) * p.H + h) * p.Nq + u % p.Nq];
  for (int m = tid; m < N; m += 128) sp[m] = p.ws_sorted[row * N + m];
  __syncthreads();
  // Exclusive prefixes in place. When every weight is 0 or at least 2^-29 and they sum below 2,
  // all of them and every partial sum are multiples of 2^-52 below 2, so each double sum is exact
  // whatever the order: wave 0 then forms them as a scan (lane L holds slots 8L .. 8L + 7) and gets
  // the sequential sum's values bit for bit. Otherwise (or past 512 slots) lane 0 runs the
  // sequential sum.
  if (w == 0) {
    bool fast = N <= 512;
    float v[8];
    double part = 0.0;
    if (fast) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int m = lane * 8 + e;
        v[e] = m < N ? sp[m] : 0.f;
        part += (double)v[e];
      }
      bool ok = true;
#pragma unroll
      for (int e = 0; e < 8; ++e) ok = ok && (v[e] == 0.f || v[e] >= 0x1p-29f);
      double incl = part;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      ok = ok && __shfl(incl, 63, 64) < 2.0;
      fast = __all(ok);
      if (fast) {
        double c = incl - part;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          c += (double)v[e];
          const int m = lane * 8 + e;
          if (m < N) sp[m] = wa_sub_rn((float)c, v[e]);
        }
      }
    }
    if (!fast && lane == 0) {
      constexpr int BATCH = 16;
      double c = 0.0;
      int m = 0;
      for (; m + BATCH <= N; m += BATCH) {
        float u[BATCH];
#pragma unroll
        for (int e = 0; e < BATCH; ++e) u[e] = sp[m + e];
#pragma unroll
        for (int e = 0; e < BATCH; ++e) {
          c += (double)u[e];
          u[e] = wa_sub_rn((float)c, u[e]);
        }
#pragma unroll
        for (int e = 0; e < BATCH; ++e) sp[m + e] = u[e];
      }
      for (; m < N; ++m) {
        const float pm = sp[m];
        c += (double)pm;
        sp[m] = wa_sub_rn((float)c, pm);
      }
    }
  }
  {
    // the head's mean Gini in the reference's fp32 order, its independent cascades on wave 1
    // (threads 64 .. 95) while thread 0 runs the prefix sum above, then the threshold (the product
    // and the sum round separately, as the reference's two tensor operations do)
    const int HN = p.H * p.Nq;
    const float sum = staged ? tc_head_sum_wg([&](int r) { return sg[(r / HN) * p.Nq + r % p.Nq]; }, p.B, p.H, p.Nq, h,
                                              s_chain, 64)
                             : tc_head_sum_wg([&](int r) { return gw[r]; }, p.B, p.H, p.Nq, h, s_chain, 64);
    if (tid == 64) {
      const float mean = wa_div_rn(sum, (float)(p.B * p.Nq));
      const float thr = wa_add_rn(p.tau_min, wa_mul_rn(mean, p.tau_span));
      s_thr = thr;
      if (b == 0 && i == 0) p.thresholds[h] = thr;
    }
  }
  __syncthreads();
  const float thr = s_thr;
  int cnt = 0;
  uint8_t* mrow = p.mask ? p.mask + row * N : nullptr;
  const int32_t* idx_row = p.index + row * N;
  for (int m = tid; m < N; m += 128) {
    const bool keep = sp[m] < thr;
    cnt += keep;
    if (mrow) mrow[idx_row[m]] = keep ? 1 : 0;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if (lane == 0) s_cnt[w] = cnt;
  __syncthreads();
  if (tid == 0) p.num[row] = s_cnt[0] + s_cnt[1];
}

// Mask -> ascending (index, num) per row, padded with -1 (block_sparse_triton.py:20-57).
__global__ void __launch_bounds__(64) map_to_index_kernel(const uint8_t* mask, int64_t ncols,
                                                          int32_t* index, int32_t* num) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const uint8_t* mrow = mask + row * ncols;
  int32_t* irow = index + row * ncols;
  int count = 0;
  for (int64_t base = 0; base < ncols; base += 64) {
    const int64_t c = base + lane;
    const bool bit = c < ncols && mrow[c] != 0;
    const uint64_t ballot = __ballot(bit);
    const int before = __popcll(ballot & ((1ull << lane) - 1ull));
    if (bit) irow[count + before] = (int32_t)c;
    count += __popcll(ballot);
  }
  for (int64_t c = count + lane; c < ncols; c += 64) irow[c] = -1;
  if (lane == 0) num[row] = count;
}

}  // namespace

namespace {

// Kernel variant of a job: 0 bf16 x8, 1 bf16 x1, 2 fp32 x4, 3 fp32 x1 (-1: invalid job).
int pool_variant(const wa_pool_args* a) {
  const bool vec_ok = wa_aligned16(a->x);
  if (a->x_dtype == WA_BF16) {
    if (vec_ok && a->D % 8 == 0 && a->x_sb % 8 == 0 && a->x_st % 8 == 0 && a->x_sh % 8 == 0 && a->D / 8 <= 256) return 0;
    return a->D <= 256 ? 1 : -1;
  }
  if (vec_ok && a->D % 4 == 0 && a->x_sb % 4 == 0 && a->x_st % 4 == 0 && a->x_sh % 4 == 0 && a->D / 4 <= 256) return 2;
  return a->D <= 256 ? 3 : -1;
}

int pool_check(const wa_pool_args* a) {
  WA_CHECK_ARG(a && a->x && a->out, "wa_block_mean_pool: null argument");
  WA_CHECK_ARG(a->x_dtype == WA_F32 || a->x_dtype == WA_BF16, "wa_block_mean_pool: bad dtype");
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->D > 0 && a->D <= 1024 && a->block_size > 0 && a->num_blocks >= 0,
               "wa_block_mean_pool: bad sizes");
  WA_CHECK_ARG(a->first_block >= 0 && a->out_blocks >= 0, "wa_block_mean_pool: bad block range");
  const int64_t end_block = a->first_block + a->num_blocks;
  WA_CHECK_ARG(a->L <= end_block * a->block_size && a->L > (end_block - 1) * a->block_size,
               "wa_block_mean_pool: L=%lld does not end in block %lld of %lld tokens", (long long)a->L,
               (long long)(end_block - 1), (long long)a->block_size);
  WA_CHECK_ARG(a->out_blocks == 0 || a->out_blocks >= end_block, "wa_block_mean_pool: out_blocks < last block");
  WA_CHECK_ARG(pool_variant(a) >= 0, "wa_block_mean_pool: an unaligned input needs D <= 256");
  return WA_OK;
}

// One launch over jobs that share a kernel variant.
int pool_launch(const wa_pool_args* const* jobs, int n, int variant, hipStream_t s) {
  PoolJobs pj{};
  int64_t total = 0;
  size_t lds = 0;
  pj.n = 0;
  for (int i = 0; i < n; ++i) {
    const wa_pool_args* a = jobs[i];
    const int64_t nh = a->heads ? a->n_heads : a->H;
    if (a->B == 0 || nh == 0 || a->num_blocks == 0) continue;
    pj.job[pj.n] = PoolParams{a->x, a->x_sb, a->x_st, a->x_sh, a->x_dtype, (int)a->L, (int)a->H, (int)a->D,
                              (int)a->block_size, (int)a->num_blocks, a->heads, a->out, a->emulate_rounding, (int)nh,
                              (int)a->first_block,
                              (int)(a->out_blocks > 0 ? a->out_blocks : a->first_block + a->num_blocks),
                              a->store_sums};
    pj.start[pj.n] = total;
    total += nh * a->num_blocks * a->B;
    const int vec = variant == 0 ? 8 : variant == 2 ? 4 : 1;
    const int rpp = 256 / (int)(a->D / vec);
    lds = std::max(lds, (size_t)rpp * (a->D + 4) * sizeof(float));
    ++pj.n;
  }
  if (pj.n == 0) return WA_OK;
  pj.start[pj.n] = total;
  WA_CHECK_ARG(total < ((int64_t)1 << 31), "wa_block_mean_pool: too many blocks for one launch");
  const dim3 grid((unsigned)total);
  switch (variant) {
    case 0: hipLaunchKernelGGL((pool_kernel<bf16_t, 8>), grid, dim3(256), lds, s, pj); break;
    case 1: hipLaunchKernelGGL((pool_kernel<bf16_t, 1>), grid, dim3(256), lds, s, pj); break;
    case 2: hipLaunchKernelGGL((pool_kernel<float, 4>), grid, dim3(256), lds, s, pj); break;
    default: hipLaunchKernelGGL((pool_kernel<float, 1>), grid, dim3(256), lds, s, pj); break;
  }
  return wa_launch_status("block_mean_pool");
}

}  // namespace

extern "C" int wa_block_mean_pool(const wa_pool_args* a, void* stream) {
  const int rc = pool_check(a);
  if (rc != WA_OK) return rc;
  return pool_launch(&a, 1, pool_variant(a), (hipStream_t)stream);
}

extern "C" int wa_block_mean_pool_n(const wa_pool_args* jobs, int32_t n_jobs, void* stream) {
  WA_CHECK_ARG(jobs && n_jobs >= 0, "wa_block_mean_pool_n: bad job list");
  for (int i = 0; i < n_jobs; ++i) {
    const int rc = pool_check(&jobs[i]);
    if (rc != WA_OK) return rc;
  }
  // jobs of one kernel variant share a launch (up to POOL_MAX_JOBS at a time)
  bool done[64] = {};
  WA_CHECK_ARG(n_jobs <= 64, "wa_block_mean_pool_n: at most 64 jobs");
  for (int i = 0; i < n_jobs; ++i) {
    if (done[i]) continue;
    const int v = pool_variant(&jobs[i]);
    const wa_pool_args* group[POOL_MAX_JOBS];
    int g = 0;
    for (int k = i; k < n_jobs && g < POOL_MAX_JOBS; ++k) {
      if (!done[k] && pool_variant(&jobs[k]) == v) {
        group[g++] = &jobs[k];
        done[k] = true;
      }
    }
    const int rc = pool_launch(group, g, v, (hipStream_t)stream);
    if (rc != WA_OK) return rc;
  }
  return WA_OK;
}

static int64_t next_pow2(int64_t n) {
  int64_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

extern "C" int64_t wa_route_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nkv) {
  const int64_t rows = B * H * Nq;
  return ((rows * Nkv + rows) * 4 + 255) / 256 * 256;
}

namespace {
template <bool SUMS>
void route_wave_launch(const RouteParams& rp, int64_t D, int64_t Nkv, dim3 wgrid, hipStream_t s) {
  if (D == 128 && Nkv <= 256) {
    if (Nkv <= 64) hipLaunchKernelGGL((route_wave_kernel<1, 128, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
    else if (Nkv <= 128) hipLaunchKernelGGL((route_wave_kernel<2, 128, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
    else hipLaunchKernelGGL((route_wave_kernel<4, 128, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
  } else {
    if (Nkv <= 64) hipLaunchKernelGGL((route_wave_kernel<1, 0, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
    else if (Nkv <= 128) hipLaunchKernelGGL((route_wave_kernel<2, 0, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
    else if (Nkv <= 256) hipLaunchKernelGGL((route_wave_kernel<4, 0, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
    else hipLaunchKernelGGL((route_wave_kernel<8, 0, 2, SUMS>), wgrid, dim3(256), 0, s, rp);
  }
}
}  // namespace

extern "C" int wa_route(const wa_route_args* a, void* stream) {
  WA_CHECK_ARG(a && a->index && a->num, "wa_route: null output");
  WA_CHECK_ARG(a->probs || (a->q_pooled && a->k_pooled), "wa_route: need probs or pooled q/k");
  WA_CHECK_ARG(a->mode == WA_ROUTE_GINI || a->mode == WA_ROUTE_TOPK, "wa_route: bad mode");
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Nq >= 0 && a->Nkv > 0 && a->Nkv <= 4096,
               "wa_route: Nkv=%lld outside [1, 4096]", (long long)a->Nkv);
  WA_CHECK_ARG(a->probs || (a->D > 0 && a->D <= 256), "wa_route: head dim must be <= 256");
  if (a->mode == WA_ROUTE_GINI) WA_CHECK_ARG(a->workspace && a->thresholds, "wa_route: GINI needs workspace and thresholds");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || a->Nq == 0 || nh == 0) return WA_OK;
  RouteParams rp{};
  rp.probs = a->probs; rp.qp = a->q_pooled; rp.kp = a->k_pooled;
  rp.B = (int)a->B; rp.H = (int)a->H; rp.Nq = (int)a->Nq; rp.Nkv = (int)a->Nkv; rp.D = (int)a->D;
  rp.NP = (int)(next_pow2(a->Nkv) < 256 ? 256 : next_pow2(a->Nkv));
  rp.mode = a->mode; rp.tau_min = a->tau_min; rp.tau_span = a->tau_span;
  rp.scale = a->scale > 0.f ? a->scale : (float)pow((double)a->D, -0.5);
  rp.head_k = a->head_k; rp.heads = a->heads; rp.n_heads = (int)nh;
  rp.index = a->index; rp.num = a->num; rp.thresholds = a->thresholds; rp.mask = a->mask;
  rp.probs_out = a->probs_out;
  WA_CHECK_ARG(a->n_clear >= 0 && (a->n_clear == 0 || a->clear), "wa_route: clear is NULL with n_clear > 0");
  rp.clear = a->clear; rp.n_clear = a->n_clear;
  WA_CHECK_ARG(a->k_sum_len <= 0 || (a->block_size > 0 && a->k_sum_len > (a->Nkv - 1) * a->block_size &&
                                     a->k_sum_len <= a->Nkv * a->block_size && a->k_sum_len < ((int64_t)1 << 30)),
               "wa_route: k_sum_len %lld does not end in key block %lld of %lld tokens", (long long)a->k_sum_len,
               (long long)(a->Nkv - 1), (long long)a->block_size);
  rp.k_sum_len = a->k_sum_len > 0 ? (int)a->k_sum_len : 0;
  rp.Bs = (int)(a->block_size > 0 ? a->block_size : 1);
  rp.k_sum_bf16 = a->k_sum_bf16;
  rp.inv_bs = (rp.Bs & (rp.Bs - 1)) == 0 ? 1.0f / (float)rp.Bs : 0.f;
  rp.k_sum_div = rp.k_sum_len > 0 && rp.k_sum_len % rp.Bs == 0;
  WA_CHECK_ARG(a->k_pooled_blocks == 0 || a->k_pooled_blocks >= a->Nkv, "wa_route: k_pooled_blocks < Nkv");
  rp.kp_blocks = (int)(a->k_pooled_blocks > 0 ? a->k_pooled_blocks : a->Nkv);
  const int64_t rows = a->B * a->H * a->Nq;
  rp.ws_sorted = (float*)a->workspace;
  rp.ws_gini = a->workspace ? (float*)a->workspace + rows * a->Nkv : nullptr;
  dim3 grid((unsigned)a->Nq + 1, (unsigned)nh, (unsigned)a->B);  // + the clearing workgroup
  hipStream_t s = (hipStream_t)stream;
  if (a->mode == WA_ROUTE_TOPK && !a->probs && !a->probs_out && a->Nkv <= 512) {
    const dim3 wgrid((unsigned)((a->Nq + 1) / 2) + 1, (unsigned)nh, (unsigned)a->B);
    if (rp.k_sum_len > 0) route_wave_launch<true>(rp, a->D, a->Nkv, wgrid, s);
    else route_wave_launch<false>(rp, a->D, a->Nkv, wgrid, s);
    return wa_launch_status("route_wave");
  }
  hipLaunchKernelGGL(route_kernel, grid, dim3(256), (size_t)rp.NP * sizeof(uint64_t), s, rp);
  int rc = wa_launch_status("route");
  if (rc != WA_OK || a->mode != WA_ROUTE_GINI) return rc;
  const int64_t staged = a->B * a->Nq <= GINI_STAGE_MAX ? a->B * a->Nq : 0;
  hipLaunchKernelGGL(gini_count_kernel, dim3((unsigned)a->Nq, (unsigned)nh, (unsigned)a->B), dim3(128),
                     (size_t)(a->Nkv + staged) * sizeof(float), s, rp);
  return wa_launch_status("route_gini_count");
}

extern "C" int wa_map_to_index(const uint8_t* mask, int64_t rows, int64_t ncols, int32_t* index,
                               int32_t* num, void* stream) {
  WA_CHECK_ARG(mask && index && num, "wa_map_to_index: null argument");
  WA_CHECK_ARG(rows >= 0 && ncols >= 0 && rows < ((int64_t)1 << 31), "wa_map_to_index: bad sizes");
  if (rows == 0) return WA_OK;
  hipLaunchKernelGGL(map_to_index_kernel, dim3((unsigned)rows), dim3(64), 0, (hipStream_t)stream, mask,
                     ncols, index, num);
  return wa_launch_status("map_to_index");
}
