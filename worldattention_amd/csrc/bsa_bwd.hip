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
//   pre   — delta per query row and a compact bf16 copy of dO ([B, heads, Lq, D]) for the streams;
//   k2q   — per (batch, head, key block) the ascending list of query blocks that listed it, with
//           multiplicity (the transposed routing of block_sparse_triton.py:364);
//   dq    — one workgroup per query block walks its key list (64-key steps, K/V streamed to LDS);
//   dkdv  — one workgroup per key block walks its query list (64-query steps, Q/dO streamed).
// Lanes own one column of every 32x32 score tile, so row statistics are per lane and the
// probabilities / score gradients feed the next product straight from the accumulators.
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
  float scale, scale_log2;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int dq_acc;
  float* dk; int64_t dk_sb, dk_st, dk_sh; int dk_acc;
  float* dv; int64_t dv_sb, dv_st, dv_sh; int dv_acc;
  // workspace
  float* delta;      // [B, n_heads, Lq]
  bf16_t* dob;       // [B, n_heads, Lq, D]
  int32_t* k2q;      // [B, n_heads, Nkv, Nq]: (query block) | (multiplicity << 16)
  int32_t* k2q_num;  // [B, n_heads, Nkv]
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
  if (qi < p.Lq && threadIdx.x % TPR == 0) p.delta[((int64_t)b * p.n_heads + hs) * p.Lq + qi] = s;
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

// ---------------------------------------------------------------------------------------------
// dq: one workgroup (BS / 32 waves, wave w = query rows 32w..) per (batch, head slot, query
// block); 64-key steps over the row's list, K and V streamed to a double-buffered LDS tile.
// ---------------------------------------------------------------------------------------------
template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) bwd_dq_kernel(BwdParams p) {
  constexpr int NW = BS / 32, DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D;
  __shared__ __attribute__((aligned(1024))) bf16_t k0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t v0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t k1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t v1[TILE];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int qb = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int64_t irow = ((int64_t)b * p.H + h) * p.Nq + qb;
  const int n = row_visits(p, irow);
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  const int64_t srow = ((int64_t)b * p.n_heads + hs) * p.Lq;

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
  const float lse2 = q_ok ? p.lse[((int64_t)b * p.H + h) * p.Lq + qi] * WA_LOG2E : 0.f;
  const float dl = q_ok ? p.delta[srow + qi] : 0.f;
  // a row with no finite logsumexp (empty list) has zero gradients
  const bool live = q_ok && lse2 > -INFINITY;

  f32x16 dqacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dqacc[t] = f32x16{};

  const bf16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const int32_t* lst = p.index ? p.index + irow * p.index_width : nullptr;
  // steps: visit s, half hf (BS = 128 blocks have two 64-key halves)
  constexpr int HPV = BS / 64;
  const int total = n * HPV;
  auto step_info = [&](int t, int& j, int& real) {
    const int s = t / HPV, hf = t % HPV;
    j = lst ? min(max(lst[s], 0), p.Nkv - 1) : s;
    real = kv_real(p, j, BS) - 64 * hf;
    return (int64_t)j * BS + 64 * hf;
  };
  if (total > 0) {
    int j, real;
    const int64_t r0 = step_info(0, j, real);
    if (real > 0) {
      tile_dma<D, NW>(k0, kbase + r0 * p.k_st, p.k_st, real, w, lane);
      tile_dma<D, NW>(v0, vbase + r0 * p.v_st, p.v_st, real, w, lane);
    }
  }
  for (int t = 0; t < total; ++t) {
    int j, real;
    step_info(t, j, real);
    bf16_t* kc = (t & 1) ? k1 : k0;
    bf16_t* vc = (t & 1) ? v1 : v0;
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (t + 1 < total) {
      int jn, rn;
      const int64_t r0 = step_info(t + 1, jn, rn);
      if (rn > 0) {
        tile_dma<D, NW>((t & 1) ? k0 : k1, kbase + r0 * p.k_st, p.k_st, rn, w, lane);
        tile_dma<D, NW>((t & 1) ? v0 : v1, vbase + r0 * p.v_st, p.v_st, rn, w, lane);
      }
    }
    if (real <= 0) continue;  // uniform: an empty half contributes nothing
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
    // dS^T = P^T (dP^T - delta), packed in accumulator order for the next product
    bf16x8 dsb[4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        float pr = __builtin_amdgcn_exp2f(fmaf(sacc[kt][r], p.scale_log2, -lse2));
        if (key >= real || !live) pr = 0.f;
        dsb[kt * 2 + (r >> 3)][r & 7] = (bf16_t)(pr * (pacc[kt][r] - dl));
      }
    }
    // dQ[q, d] += dS[q, key] K[key, d]: A = dS (registers), B = K (transpose reads)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int tt = 0; tt < DT; ++tt) dqacc[tt] = wa_mfma32(dsb[c], tile_tr8<D>(kc, c, 32 * tt, lane), dqacc[tt]);
    }
  }
  // accumulator lane (d = 32t + l32, g) holds rows q = 32w + 8(r/4) + 4g + r%4. With accumulation
  // every previous value of a tile is read before any store, so the reads overlap (a store may
  // alias a later read, which would otherwise serialize each read-add-write round trip).
  float* dq_col = p.dq + (int64_t)b * p.dq_sb + (int64_t)h * p.dq_sh + l32;
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
// dkdv: one workgroup (BS / 32 waves, wave w = keys 32w..) per (batch, head slot, key block);
// 64-query steps over the query blocks that listed it, Q and dO streamed to LDS.
// ---------------------------------------------------------------------------------------------
template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) bwd_dkdv_kernel(BwdParams p) {
  constexpr int NW = BS / 32, DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D;
  constexpr int QPB = BS / 64;  // 64-query steps per query block
  __shared__ __attribute__((aligned(1024))) bf16_t q0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t d0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t q1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t d1[TILE];
  __shared__ float st_lse[2][64], st_dl[2][64];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int j = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = head_of(p, hs);
  if (h < 0 || h >= p.H) return;
  const int real = kv_real(p, j, BS);
  const int key = w * 32 + l32;  // this lane's key within the block
  const bool k_ok = key < real;
  const int64_t srow = ((int64_t)b * p.n_heads + hs) * p.Lq;
  const int32_t* lst = p.k2q + (((int64_t)b * p.n_heads + hs) * p.Nkv + j) * p.Nq;
  const int nl = p.k2q_num[((int64_t)b * p.n_heads + hs) * p.Nkv + j];

  // K^T and V^T fragments (B operands): lane holds row `key`, channels 16c + 8g .. +8
  bf16x8 kf[DC], vf[DC];
  {
    const int kr = j * BS + (k_ok ? key : 0);
    const bf16_t* kp = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + (int64_t)kr * p.k_st;
    const bf16_t* vp = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + (int64_t)kr * p.v_st;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const bf16x8 a = *(const bf16x8*)(kp + c * 16 + g * 8);
      const bf16x8 d = *(const bf16x8*)(vp + c * 16 + g * 8);
      kf[c] = k_ok ? a : bf16x8{};
      vf[c] = k_ok ? d : bf16x8{};
    }
  }
  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dkacc[t] = dvacc[t] = f32x16{};

  const bf16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const bf16_t* dbase = p.dob + srow * D;
  const int total = nl * QPB;
  auto issue = [&](int t, bf16_t* ql, bf16_t* dl, int buf) {
    const int e = lst[t / QPB];
    const int i = e & 0xFFFF;
    const int q0r = i * BS + 64 * (t % QPB);
    const int rq = min(64, p.Lq - q0r);
    if (rq > 0) {
      tile_dma<D, NW>(ql, qbase + (int64_t)q0r * p.q_st, p.q_st, rq, w, lane);
      tile_dma<D, NW>(dl, dbase + (int64_t)q0r * D, D, rq, w, lane);
    }
    for (int r = tid; r < 64; r += 2 * BS) {
      const int qq = q0r + r;
      const float lv = qq < p.Lq ? p.lse[((int64_t)b * p.H + h) * p.Lq + qq] * WA_LOG2E : -INFINITY;
      st_lse[buf][r] = lv;
      st_dl[buf][r] = qq < p.Lq ? p.delta[srow + qq] : 0.f;
    }
  };
  if (total > 0) issue(0, q0, d0, 0);
  for (int t = 0; t < total; ++t) {
    const int e = lst[t / QPB];
    const float mult = (float)(e >> 16);
    const int q0r = (e & 0xFFFF) * BS + 64 * (t % QPB);
    const int buf = t & 1;
    bf16_t* qc = buf ? q1 : q0;
    bf16_t* dc = buf ? d1 : d0;
    // the statistics of step t were written with plain LDS stores by other waves: the barrier
    // below (after their lgkm wait) publishes them together with the streamed tiles
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t + 1 < total) issue(t + 1, buf ? q0 : q1, buf ? d0 : d1, buf ^ 1);
    if (q0r >= p.Lq) continue;
    // S[q, key] = Q K^T and dP[q, key] = dO V^T per 32-query tile (A from LDS, B from registers)
    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) sacc[qt] = pacc[qt] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        sacc[qt] = wa_mfma32(tile_row8<D>(qc, qt * 32 + l32, 2 * c + g), kf[c], sacc[qt]);
        pacc[qt] = wa_mfma32(tile_row8<D>(dc, qt * 32 + l32, 2 * c + g), vf[c], pacc[qt]);
      }
    }
    // P and dS in accumulator order (lane = key, registers = queries), scaled by multiplicity
    bf16x8 pb[4], dsb[4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql = qt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float lv = st_lse[buf][ql];
        float pr = lv > -INFINITY ? __builtin_amdgcn_exp2f(fmaf(sacc[qt][r], p.scale_log2, -lv)) : 0.f;
        if (!k_ok) pr = 0.f;
        pb[qt * 2 + (r >> 3)][r & 7] = (bf16_t)(pr * mult);
        dsb[qt * 2 + (r >> 3)][r & 7] = (bf16_t)(pr * mult * (pacc[qt][r] - st_dl[buf][ql]));
      }
    }
    // dV[key, d] += P^T dO, dK[key, d] += dS^T Q: A from registers, B by transpose reads
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int tt = 0; tt < DT; ++tt) {
        dvacc[tt] = wa_mfma32(pb[c], tile_tr8<D>(dc, c, 32 * tt, lane), dvacc[tt]);
        dkacc[tt] = wa_mfma32(dsb[c], tile_tr8<D>(qc, c, 32 * tt, lane), dkacc[tt]);
      }
    }
  }
  // accumulator lane (d = 32t + l32, g) holds keys 32w + 8(r/4) + 4g + r%4; previous values of a
  // tile are all read before any store (see the dq epilogue)
  float* dk_col = p.dk + (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh + l32;
  float* dv_col = p.dv + (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh + l32;
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
    float pk[16], pv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = j * BS + w * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      const bool in = row < p.Lkv;
      pk[r] = p.dk_acc && in ? dk_col[(int64_t)row * p.dk_st + 32 * tt] : 0.f;
      pv[r] = p.dv_acc && in ? dv_col[(int64_t)row * p.dv_st + 32 * tt] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = w * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
      const int row = j * BS + kk;
      if (row < p.Lkv) {
        const bool kval = kk < real;
        dk_col[(int64_t)row * p.dk_st + 32 * tt] = pk[r] + (kval ? dkacc[tt][r] * p.scale : 0.f);
        dv_col[(int64_t)row * p.dv_st + 32 * tt] = pv[r] + (kval ? dvacc[tt][r] : 0.f);
      }
    }
  }
}

template <int D, int BS>
int launch_bwd(const BwdParams& bp, hipStream_t s) {
  const int nh = bp.n_heads;
  hipLaunchKernelGGL((bwd_pre_kernel<D>), dim3((unsigned)((bp.Lq + (256 / (D / 8)) - 1) / (256 / (D / 8))), nh, bp.B),
                     dim3(256), 0, s, bp);
  int rc = wa_launch_status("bsa_bwd_pre");
  if (rc) return rc;
  hipLaunchKernelGGL(k2q_kernel, dim3((bp.Nkv + 255) / 256, nh, bp.B), dim3(256), 0, s, bp);
  if ((rc = wa_launch_status("bsa_bwd_k2q"))) return rc;
  if (bp.dq) {
    hipLaunchKernelGGL((bwd_dq_kernel<D, BS>), dim3(bp.Nq, nh, bp.B), dim3(2 * BS), 0, s, bp);
    if ((rc = wa_launch_status("bsa_bwd_dq"))) return rc;
  }
  if (bp.dk && bp.dv) {
    hipLaunchKernelGGL((bwd_dkdv_kernel<D, BS>), dim3(bp.Nkv, nh, bp.B), dim3(2 * BS), 0, s, bp);
    if ((rc = wa_launch_status("bsa_bwd_dkdv"))) return rc;
  }
  return WA_OK;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace

extern "C" int64_t wa_bsa_bwd_workspace_bytes(int64_t B, int64_t n_heads, int64_t Lq, int64_t Lkv, int64_t D,
                                              int64_t block_size) {
  const int64_t nq = (Lq + block_size - 1) / block_size, nkv = (Lkv + block_size - 1) / block_size;
  return align256(B * n_heads * Lq * 4) + align256(B * n_heads * Lq * D * 2) +
         align256(B * n_heads * nkv * nq * 4) + align256(B * n_heads * nkv * 4);
}

extern "C" int wa_bsa_bwd(const wa_bsa_bwd_args* a, void* stream) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_bwd: null args");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_bsa_bwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_bsa_bwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq > 0 && a->Lkv > 0, "wa_bsa_bwd: bad sizes");
  WA_CHECK_ARG(a->q && a->k && a->v && a->o && a->dout && a->lse && a->workspace, "wa_bsa_bwd: null tensor");
  WA_CHECK_ARG(a->dq || (a->dk && a->dv), "wa_bsa_bwd: nothing to compute");
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
  bp.scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->D);
  bp.scale_log2 = bp.scale * WA_LOG2E;
  bp.dq = a->dq; bp.dq_sb = a->dq_sb; bp.dq_st = a->dq_st; bp.dq_sh = a->dq_sh; bp.dq_acc = a->dq_accumulate;
  bp.dk = a->dk; bp.dk_sb = a->dk_sb; bp.dk_st = a->dk_st; bp.dk_sh = a->dk_sh; bp.dk_acc = a->dk_accumulate;
  bp.dv = a->dv; bp.dv_sb = a->dv_sb; bp.dv_st = a->dv_st; bp.dv_sh = a->dv_sh; bp.dv_acc = a->dv_accumulate;
  char* ws = (char*)a->workspace;
  bp.delta = (float*)ws;
  ws += align256(a->B * nh * a->Lq * 4);
  bp.dob = (bf16_t*)ws;
  ws += align256(a->B * nh * a->Lq * a->D * 2);
  bp.k2q = (int32_t*)ws;
  ws += align256(a->B * nh * nkv * nq * 4);
  bp.k2q_num = (int32_t*)ws;

  hipStream_t s = (hipStream_t)stream;
  if (a->D == 64 && a->block_size == 64) return launch_bwd<64, 64>(bp, s);
  if (a->D == 64 && a->block_size == 128) return launch_bwd<64, 128>(bp, s);
  if (a->D == 128 && a->block_size == 64) return launch_bwd<128, 64>(bp, s);
  return launch_bwd<128, 128>(bp, s);
}
