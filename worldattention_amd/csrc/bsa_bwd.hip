// Block-sparse flash-attention backward for gfx950 (bf16 MFMA 32x32x16, fp32 accumulation).
//
// Reference semantics: the gradient of block_sparse_attention_reference
// (wan/modules/hsa/block_sparse_torch.py:16-64) under autograd — listed key blocks in any order,
// ids clamped, a block listed twice contributes twice, masked keys and empty rows contribute
// nothing — which is what the Triton backward (block_sparse_triton.py:142-368) computes for
// square problems. Here Lq and Lkv are independent (the Triton kernel assumes Lq == Lkv).
//
//   P = exp(S scale - lse),  dP = dO V^T,  dS = P (dP - delta),  delta = rowsum(O * dO)
//   dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO
//
// Kernels:
//   pre   — per query row delta and the base-2 log-sum-exp (+inf for a row without one, so that
//           its probabilities come out 0), and a compact bf16 copy of dO ([B, heads, Lq, D]);
//   k2q   — per (batch, head, key block) the ascending list of query blocks that listed it, with
//           multiplicity (the transposed routing of block_sparse_triton.py:364);
//   dq    — one workgroup per query block walks its key list (64-key steps, K/V streamed to LDS);
//   dkdv  — one workgroup per 64 keys of a key block walks the block's query list (64-query
//           steps, Q/dO streamed).
// Lanes own one column of every 32x32 score tile, so row statistics are per lane and the
// probabilities / score gradients feed the next product straight from the accumulators.
#include <algorithm>
#include <type_traits>

#include "tile.h"

namespace {

struct BwdParams {
  const bf16_t* q; int64_t q_sb, q_st, q_sh;
  const bf16_t* k; int64_t k_sb, k_st, k_sh;
  const bf16_t* v; int64_t v_sb, v_st, v_sh;
  const void* o; int64_t o_sb, o_st, o_sh; int o_dtype;
  const void* dout; int64_t d_sb, d_st, d_sh; int d_dtype;
  const float* lse;                       // [B, H, Lq], natural log
  const int32_t* index; const int32_t* num; int64_t index_width;
  const int32_t* block_sizes;
  const int32_t* heads; int n_heads;
  int B, H, Lq, Lkv, Nq, Nkv;
  int64_t q_slab, k_slab, v_slab;  // bytes of one (batch, head) Q / K / V slab: first row to last row's end
  float scale, scale_log2;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int dq_acc;
  int dq_bf16;   // dq is bf16 (written once, rounded from the fp32 result) instead of fp32
  void* dk; int64_t dk_sb, dk_st, dk_sh; int dk_acc;
  void* dv; int64_t dv_sb, dv_st, dv_sh; int dv_acc;
  int dkv_bf16;  // dk / dv are bf16 (written once) instead of fp32
  int dkv_vec;   // ... with 16-byte aligned rows: written through an LDS staging tile
  // workspace
  float* delta;      // [B, n_heads, Lq]
  float* lse2;       // [B, n_heads, Lq]: lse * log2(e), +inf where lse = -inf
  bf16_t* dob;       // [B, n_heads, Lq, D]
  int32_t* k2q;      // [B, n_heads, Nkv, Nq]: (query block) | (multiplicity << 16)
  int32_t* k2q_num;  // [B, n_heads, Nkv]
  int4* kv_info;     // [B * n_heads * Nkv] dkdv launch order: per slab, key blocks by descending list
                     // length as {block id, list length, first list entry, 0}
};

__device__ __forceinline__ int head_of(const BwdParams& p, int hs) { return p.heads ? p.heads[hs] : hs; }

__device__ __forceinline__ int row_visits(const BwdParams& p, int64_t irow) {
  if (!p.index) return p.Nkv;
  return max(0, min(p.num[irow], (int)p.index_width));
}

__device__ __forceinline__ int kv_real(const BwdParams& p, int j, int BS) {
  int real = BS;
  if (p.block_sizes) real = min(real, p.block_sizes[j]);
  return max(0, min(real, p.Lkv - j * BS));
}

__device__ __forceinline__ float load_any(const void* base, int64_t i, int dtype) {
  return dtype == WA_BF16 ? (float)((const bf16_t*)base)[i] : ((const float*)base)[i];
}

// ---------------------------------------------------------------------------------------------
// pre: 16 threads per query row (8 channels each).
// ---------------------------------------------------------------------------------------------
// O and dO rows loaded 8 elements at a time (16-byte aligned rows; the host checks, and otherwise
// launches bwd_pre_kernel, which loads element by element).
template <typename T>
__device__ __forceinline__ void load8(const void* base, int64_t i, float (&f)[8]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 v = *(const bf16x8*)((const bf16_t*)base + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
  } else {
    const f32x4 a = *(const f32x4*)((const float*)base + i), c = *(const f32x4*)((const float*)base + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = a[e];
      f[e + 4] = c[e];
    }
  }
}

template <int D, typename OT, typename DTY>
__global__ void __launch_bounds__(256) bwd_pre_vec_kernel(BwdParams p) {
  constexpr int TPR = D / 8;
  const int hs = blockIdx.y, b = blockIdx.z;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int qi = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int c0 = (threadIdx.x % TPR) * 8;
  float s = 0.f;
  float l = 0.f;
  if (qi < p.Lq) {
    const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh + c0;
    const int64_t dd = (int64_t)b * p.d_sb + (int64_t)qi * p.d_st + (int64_t)h * p.d_sh + c0;
    float ov[8], dv[8];
    load8<OT>(p.o, oo, ov);
    load8<DTY>(p.dout, dd, dv);
    if (threadIdx.x % TPR == 0) l = p.lse[((int64_t)b * p.H + h) * p.Lq + qi];
    bf16x8 db;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s = fmaf(ov[e], dv[e], s);
      db[e] = (bf16_t)dv[e];
    }
    *(bf16x8*)(p.dob + (((int64_t)b * p.n_heads + hs) * p.Lq + qi) * D + c0) = db;
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (qi < p.Lq && threadIdx.x % TPR == 0) {
    const int64_t r = ((int64_t)b * p.n_heads + hs) * p.Lq + qi;
    p.delta[r] = s;
    p.lse2[r] = l > -INFINITY ? l * WA_LOG2E : INFINITY;
  }
}

template <int D>
__global__ void __launch_bounds__(256) bwd_pre_kernel(BwdParams p) {
  constexpr int TPR = D / 8;
  const int hs = blockIdx.y, b = blockIdx.z;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int qi = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int c0 = (threadIdx.x % TPR) * 8;
  float s = 0.f;
  if (qi < p.Lq) {
    const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh + c0;
    const int64_t dd = (int64_t)b * p.d_sb + (int64_t)qi * p.d_st + (int64_t)h * p.d_sh + c0;
    bf16x8 db;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float dv = load_any(p.dout, dd + e, p.d_dtype);
      s = fmaf(load_any(p.o, oo + e, p.o_dtype), dv, s);
      db[e] = (bf16_t)dv;
    }
    *(bf16x8*)(p.dob + (((int64_t)b * p.n_heads + hs) * p.Lq + qi) * D + c0) = db;
  }
#pragma unroll
  for (int m = TPR / 2; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (qi < p.Lq && threadIdx.x % TPR == 0) {
    const int64_t r = ((int64_t)b * p.n_heads + hs) * p.Lq + qi;
    const float l = p.lse[((int64_t)b * p.H + h) * p.Lq + qi];
    p.delta[r] = s;
    p.lse2[r] = l > -INFINITY ? l * WA_LOG2E : INFINITY;
  }
}

// ---------------------------------------------------------------------------------------------
// k2q by counting: one workgroup per (64 key blocks, head slot, batch). Every list entry of the
// head that falls in the workgroup's key range adds 1 to cnt[key block][query block] in LDS; then
// thread j walks row j in query order and writes the non-zero counts. For Nq <= K2Q_COUNT_NQ.
// ---------------------------------------------------------------------------------------------
constexpr int K2Q_COUNT_KB = 64;
constexpr int K2Q_COUNT_NQ = 256;

__global__ void __launch_bounds__(256) k2q_count_kernel(BwdParams p) {
  __shared__ uint32_t cnt[K2Q_COUNT_KB * K2Q_COUNT_NQ];
  __shared__ int32_t s_num[K2Q_COUNT_NQ];
  const int hs = blockIdx.y, b = blockIdx.z, j0 = blockIdx.x * K2Q_COUNT_KB;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int64_t row0 = ((int64_t)b * p.H + h) * p.Nq;
  const int width = (int)p.index_width, nq = p.Nq;
  __shared__ int s_maxn;
  if (threadIdx.x == 0) s_maxn = 0;
  for (int u = threadIdx.x; u < K2Q_COUNT_KB * nq; u += 256) cnt[u] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < nq; i += 256) {
    const int n = row_visits(p, row0 + i);
    s_num[i] = n;
    atomicMax(&s_maxn, n);
  }
  __syncthreads();
  // only the listed entries: (row, slot < the longest row's count), four loads in flight per thread
  const int maxn = s_maxn, total = nq * maxn;
  for (int u0 = threadIdx.x; u0 < total; u0 += 4 * 256) {
    int jj[4], ii[4];
    bool on[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = u0 + k * 256;
      ii[k] = u / maxn;  // maxn > 0 whenever the loop runs
      on[k] = u < total && u - ii[k] * maxn < s_num[min(ii[k], nq - 1)];
      jj[k] = on[k] ? p.index[(row0 + ii[k]) * width + (u - ii[k] * maxn)] : 0;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = min(max(jj[k], 0), p.Nkv - 1) - j0;
      if (on[k] && j >= 0 && j < K2Q_COUNT_KB) atomicAdd(&cnt[j * nq + ii[k]], 1u);
    }
  }
  __syncthreads();
  const int j = j0 + (int)threadIdx.x;
  if (threadIdx.x >= K2Q_COUNT_KB || j >= p.Nkv) return;
  int32_t* out = p.k2q + (((int64_t)b * p.n_heads + hs) * p.Nkv + j) * p.Nq;
  const uint32_t* c = cnt + threadIdx.x * nq;
  int n = 0;
  for (int i = 0; i < nq; ++i) {
    const int m = (int)c[i];
    if (m > 0) out[n++] = i | (min(m, 32767) << 16);
  }
  p.k2q_num[((int64_t)b * p.n_heads + hs) * p.Nkv + j] = n;
}

// ---------------------------------------------------------------------------------------------
// k2q: one workgroup per (256 key blocks, head slot, batch). The head's row lists are staged in LDS
// once (when they fit in K2Q_LDS_INTS), then thread j scans the query rows in order for block j
// with broadcast reads.
// ---------------------------------------------------------------------------------------------
constexpr int K2Q_LDS_INTS = 12288;

__global__ void __launch_bounds__(256) k2q_kernel(BwdParams p) {
  __shared__ int32_t s_list[K2Q_LDS_INTS];
  __shared__ int32_t s_num[1024];
  const int hs = blockIdx.y, b = blockIdx.z;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int64_t row0 = ((int64_t)b * p.H + h) * p.Nq;
  const int width = p.index ? (int)p.index_width : 0;
  const bool staged = p.index && p.Nq <= 1024 && (int64_t)p.Nq * width <= K2Q_LDS_INTS;
  if (staged) {
    for (int i = threadIdx.x; i < p.Nq; i += 256) s_num[i] = row_visits(p, row0 + i);
    for (int u = threadIdx.x; u < p.Nq * width; u += 256) s_list[u] = p.index[row0 * width + u];
  }
  __syncthreads();
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= p.Nkv) return;
  int32_t* out = p.k2q + (((int64_t)b * p.n_heads + hs) * p.Nkv + j) * p.Nq;
  int cnt = 0;
  for (int i = 0; i < p.Nq; ++i) {
    int m = 0;
    if (!p.index) {
      m = 1;
    } else if (staged) {
      const int n = s_num[i];
      for (int s2 = 0; s2 < n; ++s2) m += min(max(s_list[i * width + s2], 0), p.Nkv - 1) == j;
    } else {
      const int n = row_visits(p, row0 + i);
      const int32_t* lst = p.index + (row0 + i) * width;
      for (int s2 = 0; s2 < n; ++s2) m += min(max(lst[s2], 0), p.Nkv - 1) == j;
    }
    if (m > 0) out[cnt++] = i | (min(m, 32767) << 16);
  }
  p.k2q_num[((int64_t)b * p.n_heads + hs) * p.Nkv + j] = cnt;
}

// The dq and dkdv passes stream their tiles through a ring of LDS stages: the tile of step t + 1
// streams in while step t is computed, issued into the stage step t - 1 freed. Every step issues the
// same number of loads (an empty half-block streams the slab's first rows), so the waits count
// them. Row lists (with each block's valid row count) are staged in LDS once, so the loop issues no
// other memory reads while they fit. Both passes run two waves per SIMD (up to 256 registers) as
// two workgroups per CU, each with a 2-stage ring, its staged list (and for dK/dV the P exchange)
// in half the CU's LDS: while one workgroup sets up or writes its result, the other computes.
constexpr int DQ_STAGES = 2, DQ_LIST_MAX = 1024;
constexpr int DKDV_KEYS = 64, DKDV_STAGES = 2, DKDV_LIST_MAX = 1024;

template <int N> using IC = std::integral_constant<int, N>;

// Stage S of a ring kept as its own LDS array (four at most), so that every stage address is static.
template <int S, class T>
__device__ __forceinline__ T* stage_of(T* s0, T* s1, T* s2, T* s3) {
  if constexpr (S == 0) return s0;
  else if constexpr (S == 1) return s1;
  else if constexpr (S == 2) return s2;
  else return s3;
}

// Top of a step: this wave's loads of the current tile are done (at most `ahead` later tiles of
// PER loads each still in flight) and so are its LDS reads of the previous step; the barrier
// extends both to the workgroup, after which the previous step's stage may be refilled.
template <int PER>
__device__ __forceinline__ void ring_wait(int ahead) {
  if (ahead >= 2) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * PER) : "memory");
  else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(PER) : "memory");
  else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------------------------
// dq: one workgroup (BS / 32 waves, wave w = query rows 32w..) per (batch, head slot, query
// block); 64-key steps over the row's list, K and V streamed through the ring.
// ---------------------------------------------------------------------------------------------
template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) __attribute__((amdgpu_waves_per_eu(2))) bwd_dq_kernel(BwdParams p) {
  constexpr int NW = BS / 32, DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D, ST = DQ_STAGES, LM = DQ_LIST_MAX;
  using TS = TileStream<D, NW>;
  constexpr int PER = 2 * TS::NI;                  // loads per wave per step: K and V
  constexpr int HPV = BS / 64;                     // 64-key steps per visited block
  constexpr int XS = ST == 4 ? 2 * TILE : 8;      // stages 2 and 3 exist only in 4-stage rings
  // stage s: K tile at [0, TILE), V tile at [TILE, 2 TILE)
  __shared__ __attribute__((aligned(1024))) bf16_t kv0[2 * TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t kv1[2 * TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t kv2[XS];
  __shared__ __attribute__((aligned(1024))) bf16_t kv3[XS];
  __shared__ int32_t s_lst[LM];  // visited block | (its valid key count << 16)
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  // 1-D grid over (batch, head slot, query block), taken XCD by XCD (wa_xcd_remap): an XCD runs
  // a contiguous run of whole slabs, so the query blocks of a head share its K / V tiles in one L2
  const int pos = wa_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int qb = pos % p.Nq, hs = (pos / p.Nq) % p.n_heads, b = pos / (p.Nq * p.n_heads);
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int64_t irow = ((int64_t)b * p.H + h) * p.Nq + qb;
  const int n = row_visits(p, irow);
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  const int64_t srow = ((int64_t)b * p.n_heads + hs) * p.Lq;

  const int32_t* lst = p.index ? p.index + irow * p.index_width : nullptr;
  auto visit = [&](int s2) {
    const int j = lst ? min(max(lst[s2], 0), p.Nkv - 1) : s2;
    return j | (kv_real(p, j, BS) << 16);
  };
  for (int i = tid; i < min(n, LM); i += 2 * BS) s_lst[i] = visit(i);
  bf16x8 qf[DC], dof[DC];
  {
    const bf16_t* qr = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok ? qi : 0) * p.q_st;
    const bf16_t* dr = p.dob + (srow + (q_ok ? qi : 0)) * D;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const bf16x8 a = *(const bf16x8*)(qr + c * 16 + g * 8);
      const bf16x8 d = *(const bf16x8*)(dr + c * 16 + g * 8);
      qf[c] = q_ok ? a : bf16x8{};
      dof[c] = q_ok ? d : bf16x8{};
    }
  }
  // a query past Lq or without a log-sum-exp gets lse2 = +inf: zero probabilities, zero gradient
  float lse2 = q_ok ? p.lse2[srow + qi] : INFINITY;
  float dl = q_ok ? p.delta[srow + qi] : 0.f;
  // materialize the fragments before the ring's loads are issued: a use after the prologue would
  // otherwise wait for every load in flight
#pragma unroll
  for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]), "+v"(dof[c]));
  asm volatile("" : "+v"(lse2), "+v"(dl));
  __syncthreads();  // s_lst

  f32x16 dqacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dqacc[t] = f32x16{};

  TS ks, vs;
  ks.init(p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh, p.k_st, p.k_slab, w, lane);
  vs.init(p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh, p.v_st, p.v_slab, w, lane);
  const int total = n * HPV;
  // step t = (visit t / HPV, half t % HPV): first key row and real key count (<= 0: empty half)
  // (an empty half streams rows from key 0: never read, keeps the load count uniform)
  auto step_at = [&](int t, int& real) -> int {
    const int s2 = t / HPV, hf = t % HPV;
    const int e = __builtin_amdgcn_readfirstlane(s2 < LM ? s_lst[s2] : visit(s2));
    real = (e >> 16) - 64 * hf;
    return real > 0 ? (e & 0xFFFF) * BS + 64 * hf : 0;
  };
  auto issue = [&](auto S, int t) {
    bf16_t* kv = stage_of<decltype(S)::value>(kv0, kv1, kv2, kv3);
    int real;
    const int r0 = step_at(t, real);
    ks.issue(kv, r0, w);
    vs.issue(kv + TILE, r0, w);
  };
  // step t computes on stage t % ST; the loop is unrolled by ST so that every stage is static
  auto step = [&](auto S, int t) {
    constexpr int SV = decltype(S)::value;
    ring_wait<PER>(min(ST - 2, total - 1 - t));
    if (t + ST - 1 < total) issue(IC<(SV + ST - 1) % ST>{}, t + ST - 1);  // the stage of step t - 1
    int real;
    step_at(t, real);
    if (real <= 0) return;  // uniform: an empty half contributes nothing
    const bf16_t* kc = stage_of<SV>(kv0, kv1, kv2, kv3);
    const bf16_t* vc = kc + TILE;
    // S^T = K Q^T and dP^T = V dO^T (A from LDS, B from registers)
    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) sacc[kt] = pacc[kt] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        sacc[kt] = wa_mfma32(tile_row8<D>(kc, kt * 32 + l32, 2 * c + g), qf[c], sacc[kt]);
        pacc[kt] = wa_mfma32(tile_row8<D>(vc, kt * 32 + l32, 2 * c + g), dof[c], pacc[kt]);
      }
    }
    // keys past a partial block's end (their tile rows hold other keys) get zero probability
    if (real < 64) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= real) sacc[kt][r] = -INFINITY;
        }
      }
    }
    // dS^T = P^T (dP^T - delta), packed in accumulator order for the next product
    bf16x8 dsb[4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(fmaf(sacc[kt][r], p.scale_log2, -lse2));
        dsb[kt * 2 + (r >> 3)][r & 7] = (bf16_t)(pr * (pacc[kt][r] - dl));
      }
    }
    // dQ[q, d] += dS[q, key] K[key, d]: A = dS (registers), B = K (transpose reads)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int tt = 0; tt < DT; ++tt) dqacc[tt] = wa_mfma32(dsb[c], tile_tr8<D>(kc, c, 32 * tt, lane), dqacc[tt]);
    }
  };
  // prologue: tiles 0 .. ST - 2
  if (total > 0) issue(IC<0>{}, 0);
  if constexpr (ST == 4) {
    if (total > 1) issue(IC<1>{}, 1);
    if (total > 2) issue(IC<2>{}, 2);
  }
  for (int t = 0; t < total; t += ST) {
    step(IC<0>{}, t);
    if (t + 1 < total) step(IC<1>{}, t + 1);
    if constexpr (ST == 4) {
      if (t + 2 < total) step(IC<2>{}, t + 2);
      if (t + 3 < total) step(IC<3>{}, t + 3);
    }
  }
  // accumulator lane (d = 32t + l32, g) holds rows q = 32w + 8(r/4) + 4g + r%4. With accumulation
  // every previous value of a tile is read before any store, so the reads overlap (a store may
  // alias a later read, which would otherwise serialize each read-add-write round trip).
  const int64_t dq_off = (int64_t)b * p.dq_sb + (int64_t)h * p.dq_sh + l32;
  if (p.dq_bf16) {
    bf16_t* dq_out = (bf16_t*)p.dq + dq_off;
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = qb * BS + w * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (q < p.Lq) dq_out[(int64_t)q * p.dq_st + 32 * tt] = (bf16_t)(dqacc[tt][r] * p.scale);
      }
    }
    return;
  }
  float* dq_col = p.dq + dq_off;
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
    float prev[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = qb * BS + w * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      prev[r] = p.dq_acc && q < p.Lq ? dq_col[(int64_t)q * p.dq_st + 32 * tt] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = qb * BS + w * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      if (q < p.Lq) dq_col[(int64_t)q * p.dq_st + 32 * tt] = prev[r] + dqacc[tt][r] * p.scale;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// kv_order: the dkdv launch order. Workgroup s sorts the key blocks of (batch, head) slab s by
// transposed list length, longest first, into kv_info[s Nkv ..] with each block's list length and
// first list entry, so a dkdv workgroup learns all it needs for its first tiles from one load
// (a counting sort; blocks of
// equal length land in any order, which changes nothing but the schedule: every block's dK / dV is
// computed by one workgroup alone). The dkdv grid takes this order XCD by XCD (wa_xcd_remap: XCD x
// runs a contiguous run of it), so each XCD works through whole slabs, longest blocks first, and a
// slab's Q and dO tiles are fetched into one L2 instead of eight. Needs Nq < KV_ORDER_T.
// ---------------------------------------------------------------------------------------------
constexpr int KV_ORDER_T = 1024;

__global__ void __launch_bounds__(KV_ORDER_T) kv_order_kernel(BwdParams p) {
  __shared__ int hist[KV_ORDER_T];
  const int tid = threadIdx.x, n = p.Nkv, base = blockIdx.x * p.Nkv;
  const int32_t* num = p.k2q_num + base;
  hist[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += KV_ORDER_T) atomicAdd(&hist[min(max(num[i], 0), p.Nq)], 1);
  __syncthreads();
  // start[c] = number of blocks longer than c: an inclusive scan over c = Nq, Nq - 1, ..., 0
  const int c = p.Nq - tid;  // this thread's length, for tid <= Nq
  int v = c >= 0 ? hist[c] : 0;
  __syncthreads();
  hist[tid] = v;
  __syncthreads();
  for (int off = 1; off < KV_ORDER_T; off <<= 1) {
    const int add = tid >= off ? hist[tid - off] : 0;
    __syncthreads();
    hist[tid] += add;
    __syncthreads();
  }
  // hist[t] now counts the blocks of length >= Nq - t; the first slot of length c is hist[Nq - c] - count(c)
  const int first = c >= 0 ? hist[tid] - v : 0;
  __syncthreads();
  if (c >= 0) hist[c] = first;
  __syncthreads();
  for (int i = tid; i < n; i += KV_ORDER_T) {
    const int len = min(max(num[i], 0), p.Nq);
    const int e0 = len > 0 ? p.k2q[(int64_t)(base + i) * p.Nq] : 0;
    p.kv_info[base + atomicAdd(&hist[len], 1)] = int4{base + i, len, e0, 0};
  }
}

// ---------------------------------------------------------------------------------------------
// dkdv: one workgroup per (batch, head slot, key block, 64-key part: HB = BS / 64 per block);
// 64-query steps over the query blocks that listed the block; Q, dO and the rows' log-sum-exp and
// delta stream through the ring (the statistics as 4-byte direct-to-LDS loads, scaled at use). The
// parts of a block walk the same list at neighbouring grid positions, so they share the tiles in
// L2. Each 32-key group has two waves, w and w + 2:
//   the S-wave (w < 2) holds the group's K fragments and the dV accumulators: S = Q K^T,
//     P = exp2(S scale - lse2) (to LDS as fp16: 11 significant bits, 4x finer than the bf16 dS it
//     feeds), dV += P^T dO;
//   the dP-wave holds the V fragments and the dK accumulators: dP = dO V^T, then (P from LDS)
//     dS = P (dP - delta), dK += dS^T Q.
// A workgroup of four waves takes 77 KiB of LDS, so two share a CU (two waves per SIMD): one's
// set-up (the K / V fragments and first tiles, a memory round trip) and result stores run while
// the other computes, and their step barriers fall at different times.
// ---------------------------------------------------------------------------------------------
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <int D, int BS>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) bwd_dkdv_kernel(BwdParams p) {
  constexpr int KW = DKDV_KEYS, HB = BS / KW, NKG = KW / 32, NW = 2 * NKG, NT = 64 * NW, DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D, ST = DKDV_STAGES, LM = DKDV_LIST_MAX;
  constexpr int QPB = BS / 64;                     // 64-query steps per query block
  using TS = TileStream<D, NW>;
  constexpr int PER = 2 * TS::NI + 2;              // Q and dO tiles, lse and delta rows
  // stage s: Q tile at [0, TILE), dO tile at [TILE, 2 TILE), then 64 lse and 64 delta floats
  constexpr int SS = 2 * TILE + 256;
  static_assert(ST == 2 && NW == 4, "two ring stages, four waves");
  __shared__ __attribute__((aligned(1024))) bf16_t qd0[SS];
  __shared__ __attribute__((aligned(1024))) bf16_t qd1[SS];
  bf16_t* const qd2 = qd0;  // (no third or fourth stage)
  bf16_t* const qd3 = qd1;
  // P of each key group (fp16, accumulator order), register r of 32-query tile qt of lane L at
  // [group][qt][r / 4][L]: every access is 8 bytes per lane, lanes contiguous
  __shared__ __attribute__((aligned(1024))) f16x4 s_p[NKG][2][4][64];
  __shared__ int32_t s_lst[LM];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int kg = w % NKG;
  const bool swave = w < NKG;  // wave-uniform role
  // 1-D grid over (batch, head slot, key block, part): XCD by XCD through kv_info when there is
  // one (else through the slabs in order), so an XCD's workgroups share their slabs' Q and dO
  // tiles; one load gives the block, its list length and its first list entry
  const int gpos = wa_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int pos = gpos / HB, hb = gpos % HB;
  int id, nl, e0;
  if (p.kv_info) {
    const int4 inf = p.kv_info[pos];
    id = inf.x;
    nl = inf.y;
    e0 = inf.z;
  } else {
    id = pos;
    nl = min(max(p.k2q_num[id], 0), p.Nq);
    e0 = nl > 0 ? p.k2q[(int64_t)id * p.Nq] : 0;
  }
  id = __builtin_amdgcn_readfirstlane(id);
  nl = __builtin_amdgcn_readfirstlane(nl);
  e0 = __builtin_amdgcn_readfirstlane(e0);
  const int j = id % p.Nkv, hs = (id / p.Nkv) % p.n_heads, b = id / (p.Nkv * p.n_heads);
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int kb0 = j * BS + hb * KW;  // first key of this part
  if (nl == 0) {
    // no query block listed this key block: its written gradients are zero (accumulated ones
    // keep their values), with no tile streamed
    const int rows = max(0, min(KW, p.Lkv - kb0));
    constexpr int CPR = D / 8;
    const int64_t dk0 = (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh + (int64_t)kb0 * p.dk_st;
    const int64_t dv0 = (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh + (int64_t)kb0 * p.dv_st;
    if (p.dkv_vec) {
      for (int u = tid; u < rows * CPR; u += NT) {
        const int kk = u / CPR, c = u % CPR;
        *(bf16x8*)((bf16_t*)p.dk + dk0 + (int64_t)kk * p.dk_st + c * 8) = bf16x8{};
        *(bf16x8*)((bf16_t*)p.dv + dv0 + (int64_t)kk * p.dv_st + c * 8) = bf16x8{};
      }
    } else {
      for (int u = tid; u < rows * D; u += NT) {
        const int kk = u / D, c = u % D;
        if (p.dkv_bf16) {
          ((bf16_t*)p.dk)[dk0 + (int64_t)kk * p.dk_st + c] = (bf16_t)0.f;
          ((bf16_t*)p.dv)[dv0 + (int64_t)kk * p.dv_st + c] = (bf16_t)0.f;
        } else {
          if (!p.dk_acc) ((float*)p.dk)[dk0 + (int64_t)kk * p.dk_st + c] = 0.f;
          if (!p.dv_acc) ((float*)p.dv)[dv0 + (int64_t)kk * p.dv_st + c] = 0.f;
        }
      }
    }
    return;
  }
  const int real = kv_real(p, j, BS);
  const int kl = kg * 32 + l32;  // this lane's key within the part
  const int key = hb * KW + kl;  // ... and within the block
  const bool k_ok = key < real;
  const int64_t srow = ((int64_t)b * p.n_heads + hs) * p.Lq;
  const int32_t* lst = p.k2q + (((int64_t)b * p.n_heads + hs) * p.Nkv + j) * p.Nq;
  bf16x8 kvf[DC];
  f32x16 acc[DT];   // S-wave: dV^T; dP-wave: dK^T (lane = key, registers = channels)
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};

  TS qs, ds;
  qs.init(p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh, p.q_st, p.q_slab, w, lane);
  ds.init(p.dob + srow * D, D, (int64_t)p.Lq * D * 2, w, lane);
  const int total = nl * QPB;
  // list entry: (query block) | (multiplicity << 16); the first comes with the block, the rest
  // from the LDS copy, and lists longer than the copy read global memory (the empty asm keeps the
  // two reads apart: merged, they become one flat load that must wait for every direct-to-LDS
  // load in flight)
  auto entry = [&](int s2) {
    if (s2 == 0) return e0;
    if (s2 < LM) return __builtin_amdgcn_readfirstlane(s_lst[s2]);
    int e = lst[s2];
    asm volatile("" : "+v"(e));
    return __builtin_amdgcn_readfirstlane(e);
  };
  auto first_query = [&](int t) { return (entry(t / QPB) & 0xFFFF) * BS + 64 * (t % QPB); };
  // every wave streams the statistics too (identical values), so all waves count the same loads
  auto issue = [&](auto S, int t) {
    bf16_t* qd = stage_of<decltype(S)::value>(qd0, qd1, qd2, qd3);
    const int q0r = first_query(t);
    const int src0 = q0r < p.Lq ? q0r : 0;  // a half past Lq streams query 0 (never used)
    qs.issue(qd, src0, w);
    ds.issue(qd + TILE, src0, w);
    float* stats = (float*)(qd + 2 * TILE);
    row_stats_dma(stats, p.lse2 + srow + src0, p.Lq - src0, lane);
    row_stats_dma(stats + 64, p.delta + srow + src0, p.Lq - src0, lane);
  };
  // step t computes on stage t % ST; the loop is unrolled by ST so that every stage is static
  auto step = [&](auto S, int t) {
    constexpr int SV = decltype(S)::value;
    ring_wait<PER>(min(ST - 2, total - 1 - t));
    if (t + ST - 1 < total) issue(IC<(SV + ST - 1) % ST>{}, t + ST - 1);  // the stage of step t - 1
    const int e = entry(t / QPB);
    const float mult = (float)(e >> 16);
    const int q0r = (e & 0xFFFF) * BS + 64 * (t % QPB);
    if (q0r >= p.Lq) return;  // uniform over the workgroup
    const bf16_t* qc = stage_of<SV>(qd0, qd1, qd2, qd3);
    const bf16_t* dc = qc + TILE;
    const float* st_lse2 = (const float*)(qc + 2 * TILE);
    const float* st_dl = st_lse2 + 64;
    // S[q, key] = Q K^T (S-wave) or dP[q, key] = dO V^T (dP-wave) per 32-query tile (A from LDS,
    // B from registers); lane = key, registers = queries q = 32 qt + 8 rq + 4 g + i
    const bf16_t* at = swave ? qc : dc;
    f32x16 sacc[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) sacc[qt] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) sacc[qt] = wa_mfma32(tile_row8<D>(at, qt * 32 + l32, 2 * c + g), kvf[c], sacc[qt]);
    }
    // P (scaled by multiplicity) to LDS, or dS from the group's P; queries past Lq stream zero Q,
    // dO and statistics rows, so their dS and dO are 0 and they add nothing; keys past the
    // block's end are dropped by the epilogue
    bf16x8 ab[4];
    if (swave) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 l4 = *(const f32x4*)(st_lse2 + qt * 32 + 8 * rq + 4 * g);
          f32x4 p4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = rq * 4 + i;
            p4[i] = __builtin_amdgcn_exp2f(fmaf(sacc[qt][r], p.scale_log2, -l4[i])) * mult;
            ab[qt * 2 + (r >> 3)][r & 7] = (bf16_t)p4[i];
          }
          s_p[kg][qt][rq][lane] = f16x4{(_Float16)p4[0], (_Float16)p4[1], (_Float16)p4[2], (_Float16)p4[3]};
        }
      }
    }
    __syncthreads();  // P of every group in LDS
    if (!swave) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 d4 = *(const f32x4*)(st_dl + qt * 32 + 8 * rq + 4 * g);
          const f16x4 p4 = s_p[kg][qt][rq][lane];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = rq * 4 + i;
            ab[qt * 2 + (r >> 3)][r & 7] = (bf16_t)((float)p4[i] * (sacc[qt][r] - d4[i]));
          }
        }
      }
    }
    // dV^T[d, key] += dO^T P (S-wave), dK^T[d, key] += Q^T dS (dP-wave): A by transpose reads,
    // B from registers (lane = key, registers = channels d = 32 tt + 8 rq + 4 g + i)
    const bf16_t* bt = swave ? dc : qc;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int tt = 0; tt < DT; ++tt) acc[tt] = wa_mfma32(tile_tr8<D>(bt, c, 32 * tt, lane), ab[c], acc[tt]);
    }
  };
  // Set-up, all behind the one load of the block's info: the prologue tiles 0 .. ST - 2 (within
  // the first list entry's query block: no list needed), the list copy, and the K^T (S-wave) or
  // V^T (dP-wave) fragments (B operands: lane holds row `key`, channels 16c + 8g .. +8). The
  // fragments are waited for before the first step: later, the compiler (which cannot count the
  // ring's inline-assembly loads) would wait for every load in flight.
  static_assert(ST - 1 <= QPB, "the prologue tiles must come from the first list entry");
  issue(IC<0>{}, 0);
  if constexpr (ST >= 3) {
    if (total > 1) issue(IC<1>{}, 1);
  }
  for (int i = tid; i < min(nl, LM); i += NT) s_lst[i] = lst[i];
  {
    const int kr = j * BS + (k_ok ? key : 0);
    const bf16_t* src = swave ? p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + (int64_t)kr * p.k_st
                              : p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + (int64_t)kr * p.v_st;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const bf16x8 a = *(const bf16x8*)(src + c * 16 + g * 8);
      kvf[c] = k_ok ? a : bf16x8{};
    }
  }
#pragma unroll
  for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(kvf[c]));
  __syncthreads();  // s_lst
  for (int t = 0; t < total; t += ST) {
    step(IC<0>{}, t);
    if (t + 1 < total) step(IC<1>{}, t + 1);
    if constexpr (ST >= 3) {
      if (t + 2 < total) step(IC<2>{}, t + 2);
    }
    if constexpr (ST >= 4) {
      if (t + 3 < total) step(IC<3>{}, t + 3);
    }
  }
  // each lane holds its key's row: channels 32 tt + 8 rq + 4 g .. + 3 of tile tt (keys past the
  // block's end get zeros); dK is scaled here
  const float osc = swave ? 1.f : p.scale;
  if (p.dkv_vec) {
    // bf16 rows staged in the (drained) ring, row r's 16-byte chunk c at chunk c ^ swz(r): one
    // 8-byte write per (tile, rq), then 16-byte stores of whole rows
    auto swz = [](int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); };
    __syncthreads();
    bf16_t* stg = swave ? qd1 : qd0;  // dV, dK
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        bf16x4 v4;
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = (bf16_t)(k_ok ? acc[tt][rq * 4 + i] * osc : 0.f);
        *(bf16x4*)(stg + kl * D + (((4 * tt + rq) ^ swz(kl)) << 3) + 4 * g) = v4;
      }
    }
    __syncthreads();
    constexpr int CPR = D / 8;
    const int64_t dk0 = (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh;
    const int64_t dv0 = (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh;
    for (int u = tid; u < KW * CPR; u += NT) {
      const int kk = u / CPR, c = u % CPR, row = kb0 + kk;
      if (row >= p.Lkv) continue;
      const int at = kk * D + ((c ^ swz(kk)) << 3);
      *(bf16x8*)((bf16_t*)p.dk + dk0 + (int64_t)row * p.dk_st + c * 8) = *(const bf16x8*)(qd0 + at);
      *(bf16x8*)((bf16_t*)p.dv + dv0 + (int64_t)row * p.dv_st + c * 8) = *(const bf16x8*)(qd1 + at);
    }
    return;
  }
  const int row = j * BS + key;
  if (row >= p.Lkv) return;
  const int64_t o0 = (swave ? (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh + (int64_t)row * p.dv_st
                            : (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh + (int64_t)row * p.dk_st) + 4 * g;
  if (p.dkv_bf16) {
    bf16_t* dst = (bf16_t*)(swave ? p.dv : p.dk) + o0;
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dst[32 * tt + 8 * (r >> 2) + (r & 3)] = (bf16_t)(k_ok ? acc[tt][r] * osc : 0.f);
    }
    return;
  }
  // fp32: every previous value is read before any store (a load issued after a store waits for it)
  float* dst = (float*)(swave ? p.dv : p.dk) + o0;
  const int add = swave ? p.dv_acc : p.dk_acc;
  float prev[DT][16];
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) prev[tt][r] = add ? dst[32 * tt + 8 * (r >> 2) + (r & 3)] : 0.f;
  }
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      dst[32 * tt + 8 * (r >> 2) + (r & 3)] = prev[tt][r] + (k_ok ? acc[tt][r] * osc : 0.f);
  }
}

// The launches of one backward on stream s; with a second stream sq (and its fork / join events)
// the dQ pass runs on sq once the preprocess is done (it reads delta, lse2 and the bf16 dO copy, not
// the transposed lists), concurrently with the transposed lists and the dK/dV pass on s, and s
// waits for it at the end (also on an error path once forked, so a capture ends joined).
template <int D, int BS>
int launch_bwd(const BwdParams& bp, hipStream_t s, hipStream_t sq, hipEvent_t fork, hipEvent_t join) {
  const int nh = bp.n_heads;
  const dim3 pre_grid((unsigned)((bp.Lq + (256 / (D / 8)) - 1) / (256 / (D / 8))), nh, bp.B);
  // 8-element row vectors: a 16-byte aligned base and strides in multiples of 8 elements
  auto vec_ok = [](const void* ptr, int64_t sb, int64_t st, int64_t sh) {
    return wa_aligned16(ptr) && sb % 8 == 0 && st % 8 == 0 && sh % 8 == 0;
  };
  const bool ov = vec_ok(bp.o, bp.o_sb, bp.o_st, bp.o_sh);
  const bool dv = vec_ok(bp.dout, bp.d_sb, bp.d_st, bp.d_sh);
  if (ov && dv && bp.o_dtype == WA_F32 && bp.d_dtype == WA_BF16)
    hipLaunchKernelGGL((bwd_pre_vec_kernel<D, float, bf16_t>), pre_grid, dim3(256), 0, s, bp);
  else if (ov && dv && bp.o_dtype == WA_BF16 && bp.d_dtype == WA_BF16)
    hipLaunchKernelGGL((bwd_pre_vec_kernel<D, bf16_t, bf16_t>), pre_grid, dim3(256), 0, s, bp);
  else if (ov && dv && bp.o_dtype == WA_F32 && bp.d_dtype == WA_F32)
    hipLaunchKernelGGL((bwd_pre_vec_kernel<D, float, float>), pre_grid, dim3(256), 0, s, bp);
  else if (ov && dv && bp.o_dtype == WA_BF16 && bp.d_dtype == WA_F32)
    hipLaunchKernelGGL((bwd_pre_vec_kernel<D, bf16_t, float>), pre_grid, dim3(256), 0, s, bp);
  else
    hipLaunchKernelGGL((bwd_pre_kernel<D>), pre_grid, dim3(256), 0, s, bp);
  int rc = wa_launch_status("bsa_bwd_pre");
  if (rc) return rc;
  const bool split = bp.dq && sq && sq != s;
  if (split) {
    hipError_t e;
    if ((e = hipEventRecord(fork, s)) != hipSuccess || (e = hipStreamWaitEvent(sq, fork, 0)) != hipSuccess)
      return wa_fail((int)e, "wa_bsa_bwd: fork: %s", hipGetErrorString(e));
    hipLaunchKernelGGL((bwd_dq_kernel<D, BS>), dim3((unsigned)(bp.Nq * nh * bp.B)), dim3(2 * BS), 0, sq, bp);
    rc = wa_launch_status("bsa_bwd_dq");
    if ((e = hipEventRecord(join, sq)) != hipSuccess) return rc ? rc : wa_fail((int)e, "wa_bsa_bwd: join: %s", hipGetErrorString(e));
    if (rc) {
      hipStreamWaitEvent(s, join, 0);
      return rc;
    }
  }
  auto joined = [&](int code) {
    if (!split) return code;
    const hipError_t e = hipStreamWaitEvent(s, join, 0);
    return code != WA_OK ? code : e != hipSuccess ? wa_fail((int)e, "wa_bsa_bwd: join: %s", hipGetErrorString(e)) : WA_OK;
  };
  if (bp.index && bp.Nq <= K2Q_COUNT_NQ)
    hipLaunchKernelGGL(k2q_count_kernel, dim3((bp.Nkv + K2Q_COUNT_KB - 1) / K2Q_COUNT_KB, nh, bp.B), dim3(256), 0, s,
                       bp);
  else
    hipLaunchKernelGGL(k2q_kernel, dim3((bp.Nkv + 255) / 256, nh, bp.B), dim3(256), 0, s, bp);
  if ((rc = wa_launch_status("bsa_bwd_k2q"))) return joined(rc);
  if (bp.dq && !split) {
    hipLaunchKernelGGL((bwd_dq_kernel<D, BS>), dim3((unsigned)(bp.Nq * nh * bp.B)), dim3(2 * BS), 0, s, bp);
    if ((rc = wa_launch_status("bsa_bwd_dq"))) return rc;
  }
  if (bp.dk && bp.dv) {
    BwdParams kp = bp;
    if (bp.Nq < KV_ORDER_T) {
      hipLaunchKernelGGL(kv_order_kernel, dim3((unsigned)(bp.B * nh)), dim3(KV_ORDER_T), 0, s, bp);
      if ((rc = wa_launch_status("bsa_bwd_kv_order"))) return joined(rc);
    } else {
      kp.kv_info = nullptr;
    }
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, BS>), dim3((unsigned)(bp.B * nh * bp.Nkv * (BS / DKDV_KEYS))), dim3(256), 0,
                       s, kp);
    if ((rc = wa_launch_status("bsa_bwd_dkdv"))) return joined(rc);
  }
  return joined(WA_OK);
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace

extern "C" int64_t wa_bsa_bwd_workspace_bytes(int64_t B, int64_t n_heads, int64_t Lq, int64_t Lkv, int64_t D,
                                              int64_t block_size) {
  const int64_t nq = (Lq + block_size - 1) / block_size, nkv = (Lkv + block_size - 1) / block_size;
  return 2 * align256(B * n_heads * Lq * 4) + align256(B * n_heads * Lq * D * 2) +
         align256(B * n_heads * nkv * nq * 4) + align256(B * n_heads * nkv * 4) + align256(B * n_heads * nkv * 16);
}

// wa_bsa_bwd with its dQ pass on a second stream (NULL: one stream), forked from `stream` after the
// preprocess with fork_event and joined back with join_event; the one-call backward (hsa.hip) uses it.
int wa_bsa_bwd_streams(const wa_bsa_bwd_args* a, void* stream, void* dq_stream, void* fork_event, void* join_event);

extern "C" int wa_bsa_bwd(const wa_bsa_bwd_args* a, void* stream) {
  return wa_bsa_bwd_streams(a, stream, nullptr, nullptr, nullptr);
}

int wa_bsa_bwd_streams(const wa_bsa_bwd_args* a, void* stream, void* dq_stream, void* fork_event, void* join_event) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_bwd: null args");
  WA_CHECK_ARG(dq_stream == nullptr || (fork_event && join_event), "wa_bsa_bwd: a dQ stream needs fork and join events");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_bsa_bwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_bsa_bwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq > 0 && a->Lkv > 0, "wa_bsa_bwd: bad sizes");
  WA_CHECK_ARG(a->q && a->k && a->v && a->o && a->dout && a->lse && a->workspace, "wa_bsa_bwd: null tensor");
  WA_CHECK_ARG(a->dq || (a->dk && a->dv), "wa_bsa_bwd: nothing to compute");
  WA_CHECK_ARG(a->dkv_dtype == WA_F32 || (a->dkv_dtype == WA_BF16 && !a->dk_accumulate && !a->dv_accumulate),
               "wa_bsa_bwd: dkv_dtype must be WA_F32, or WA_BF16 without accumulation");
  WA_CHECK_ARG(a->dq_dtype == WA_F32 || (a->dq_dtype == WA_BF16 && !a->dq_accumulate),
               "wa_bsa_bwd: dq_dtype must be WA_F32, or WA_BF16 without accumulation");
  WA_CHECK_ARG(wa_aligned16(a->q) && wa_aligned16(a->k) && wa_aligned16(a->v) && wa_aligned16(a->workspace),
               "wa_bsa_bwd: q/k/v/workspace must be 16-byte aligned");
  WA_CHECK_ARG(a->q_sb % 8 == 0 && a->q_st % 8 == 0 && a->q_sh % 8 == 0 && a->k_sb % 8 == 0 && a->k_st % 8 == 0 &&
                   a->k_sh % 8 == 0 && a->v_sb % 8 == 0 && a->v_st % 8 == 0 && a->v_sh % 8 == 0,
               "wa_bsa_bwd: q/k/v strides must be multiples of 8 elements");
  WA_CHECK_ARG((a->o_dtype == WA_F32 || a->o_dtype == WA_BF16) && (a->dout_dtype == WA_F32 || a->dout_dtype == WA_BF16),
               "wa_bsa_bwd: bad o/dout dtype");
  if (a->index) WA_CHECK_ARG(a->num && a->index_width > 0, "wa_bsa_bwd: index needs num and width");
  const int64_t nq = (a->Lq + a->block_size - 1) / a->block_size;
  const int64_t nkv = (a->Lkv + a->block_size - 1) / a->block_size;
  WA_CHECK_ARG(nq <= 65535 && nkv <= 65535 && a->Lq < (1 << 30) && a->Lkv < (1 << 30), "wa_bsa_bwd: problem too large");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  WA_CHECK_ARG(nh >= 0 && nh <= a->H, "wa_bsa_bwd: bad head count");
  WA_CHECK_ARG(a->B * nh * nkv < ((int64_t)1 << 31) && a->B * nh * nq < ((int64_t)1 << 31),
               "wa_bsa_bwd: too many key or query blocks");
  // the tile streams address one (batch, head) slab with 32-bit byte offsets
  const int64_t q_slab = ((a->Lq - 1) * a->q_st + a->D) * 2;
  const int64_t k_slab = ((a->Lkv - 1) * a->k_st + a->D) * 2, v_slab = ((a->Lkv - 1) * a->v_st + a->D) * 2;
  WA_CHECK_ARG(q_slab < ((int64_t)1 << 31) && k_slab < ((int64_t)1 << 31) && v_slab < ((int64_t)1 << 31) &&
                   a->Lq * a->D * 2 < ((int64_t)1 << 31) && 64 * std::max({a->q_st, a->k_st, a->v_st}) < (1 << 30),
               "wa_bsa_bwd: one Q/K/V head slab must span less than 2 GiB");
  if (a->B == 0 || nh == 0) return WA_OK;

  BwdParams bp{};
  bp.q = (const bf16_t*)a->q; bp.q_sb = a->q_sb; bp.q_st = a->q_st; bp.q_sh = a->q_sh;
  bp.k = (const bf16_t*)a->k; bp.k_sb = a->k_sb; bp.k_st = a->k_st; bp.k_sh = a->k_sh;
  bp.v = (const bf16_t*)a->v; bp.v_sb = a->v_sb; bp.v_st = a->v_st; bp.v_sh = a->v_sh;
  bp.o = a->o; bp.o_sb = a->o_sb; bp.o_st = a->o_st; bp.o_sh = a->o_sh; bp.o_dtype = a->o_dtype;
  bp.dout = a->dout; bp.d_sb = a->d_sb; bp.d_st = a->d_st; bp.d_sh = a->d_sh; bp.d_dtype = a->dout_dtype;
  bp.lse = a->lse;
  bp.index = a->index; bp.num = a->num; bp.index_width = a->index_width;
  bp.block_sizes = a->block_sizes;
  bp.heads = a->heads; bp.n_heads = (int)nh;
  bp.B = (int)a->B; bp.H = (int)a->H; bp.Lq = (int)a->Lq; bp.Lkv = (int)a->Lkv; bp.Nq = (int)nq; bp.Nkv = (int)nkv;
  bp.q_slab = q_slab; bp.k_slab = k_slab; bp.v_slab = v_slab;
  bp.scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->D);
  bp.scale_log2 = bp.scale * WA_LOG2E;
  bp.dq = a->dq; bp.dq_sb = a->dq_sb; bp.dq_st = a->dq_st; bp.dq_sh = a->dq_sh; bp.dq_acc = a->dq_accumulate;
  bp.dq_bf16 = a->dq_dtype == WA_BF16;
  bp.dk = a->dk; bp.dk_sb = a->dk_sb; bp.dk_st = a->dk_st; bp.dk_sh = a->dk_sh; bp.dk_acc = a->dk_accumulate;
  bp.dv = a->dv; bp.dv_sb = a->dv_sb; bp.dv_st = a->dv_st; bp.dv_sh = a->dv_sh; bp.dv_acc = a->dv_accumulate;
  bp.dkv_bf16 = a->dkv_dtype == WA_BF16;
  bp.dkv_vec = bp.dkv_bf16 && wa_aligned16(a->dk) && wa_aligned16(a->dv) && a->dk_sb % 8 == 0 && a->dk_st % 8 == 0 &&
               a->dk_sh % 8 == 0 && a->dv_sb % 8 == 0 && a->dv_st % 8 == 0 && a->dv_sh % 8 == 0;
  char* ws = (char*)a->workspace;
  bp.delta = (float*)ws;
  ws += align256(a->B * nh * a->Lq * 4);
  bp.lse2 = (float*)ws;
  ws += align256(a->B * nh * a->Lq * 4);
  bp.dob = (bf16_t*)ws;
  ws += align256(a->B * nh * a->Lq * a->D * 2);
  bp.k2q = (int32_t*)ws;
  ws += align256(a->B * nh * nkv * nq * 4);
  bp.k2q_num = (int32_t*)ws;
  ws += align256(a->B * nh * nkv * 4);
  bp.kv_info = (int4*)ws;

  hipStream_t s = (hipStream_t)stream, sq = (hipStream_t)dq_stream;
  hipEvent_t fe = (hipEvent_t)fork_event, je = (hipEvent_t)join_event;
  if (a->D == 64 && a->block_size == 64) return launch_bwd<64, 64>(bp, s, sq, fe, je);
  if (a->D == 64 && a->block_size == 128) return launch_bwd<64, 128>(bp, s, sq, fe, je);
  if (a->D == 128 && a->block_size == 64) return launch_bwd<128, 64>(bp, s, sq, fe, je);
  return launch_bwd<128, 128>(bp, s, sq, fe, je);
}
