// Block-sparse flash-attention forward for gfx950 (bf16 MFMA 32x32x16, fp32 accumulation).
//
// Work decomposition. A "row" is one (batch, head, query block) with its list of key blocks
// index[b,h,i,0:num]. A row's list is cut into splits of `split` consecutive visits; one workgroup
// processes one (row, split) unit and writes a normalized partial output plus its log2-sum-exp to
// the workspace. A second kernel merges the partials of each row in split order, applies the
// fusion epilogue and writes the output, so every result is independent of scheduling.
//
// Unit kernel (one workgroup = BS/32 waves; wave w owns query rows [32w, 32w+32) of the block).
// Per visited key block the K and V tiles are streamed global -> LDS with direct-to-LDS loads
// (no register staging), into two separate buffers so that the next K tile streams in while the
// softmax and the PV product of the current one run. Products use the transposed formulation
//     S^T[key, q] = K[key, :] . Q[q, :]         (A = K from LDS, B = Q^T in registers)
//     O^T[d, q]  += V^T[d, key] . P^T[key, q]   (A = V^T by transpose-reads of row-major V)
// so each lane owns one query column: the row max / row sum need one exchange with lane^32 and
// the probabilities feed the PV product straight from the QK accumulator registers.
//
// LDS layouts (no padding; XOR swizzles on 16-byte chunks keep every read conflict-free):
//   K[key][chunk ^ (key & 7)]        read with ds_read_b128 (8 lanes = 8 keys, one chunk)
//   V[key][chunk ^ 2*(key & 3)]      read with ds_read_b64_tr_b16 (16 lanes = 4 keys x 32 bytes)
//
// Reference semantics: wan/modules/hsa/block_sparse_triton.py:67-139 (online softmax, partial
// trailing block mask, empty list -> 0, LSE output) and block_sparse_torch.py:16-64 (id clamping,
// listed order, duplicates attended twice, fp32 math).
#include "common.h"

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define WA_LDS(p) ((__attribute__((address_space(3))) void*)(p))
#define WA_LDS4(p) ((__attribute__((address_space(3))) s16x4*)(p))

struct FwdParams {
  const bf16_t* q; int64_t q_sb, q_st, q_sh;
  const bf16_t* k; int64_t k_sb, k_st, k_sh;
  const bf16_t* v; int64_t v_sb, v_st, v_sh;
  void* o; int64_t o_sb, o_st, o_sh; int o_dtype;
  float* lse;
  const int32_t* index; const int32_t* num; int64_t index_width;
  const int32_t* block_sizes;
  const int32_t* heads; int n_heads;
  int B, H, Lq, Lkv, Nq, Nkv;
  float scale_log2;
  int epilogue;
  const void* x; int64_t x_sb, x_st, x_sh; int x_dtype;
  const bf16_t* gate_w; const float* gate_b;
  int gate_pre_bf16, gate_out_bf16, attn_round_bf16;
  // split bookkeeping
  const int32_t* units;  // [n_units][2] = (row, split) or NULL: unit u = (u / max_splits, u % max_splits)
  int n_units, max_splits, split;
  int64_t n_rows;
  float* part_o;         // [rows * max_splits][BS][D] normalized partial outputs
  float* part_lse;       // [rows * max_splits][BS] log2-sum-exp of the partials
};

// Workgroup barrier without the global-memory fence of __syncthreads (which would wait for the
// in-flight K/V tile loads). LDS reads before it have completed: their results were consumed.
__device__ __forceinline__ void wa_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// `irow` numbers rows by global head, (b * H + h) * Nq + i: the layout of index / num. Units and
// workspace slots number rows by head slot instead, (b * n_heads + slot) * Nq + i.
__device__ __forceinline__ int row_visits(const FwdParams& p, int64_t irow) {
  if (!p.index) return p.Nkv;
  const int n = p.num[irow];
  return max(0, min(n, (int)p.index_width));
}

__device__ __forceinline__ int block_real(const FwdParams& p, int j, int BS) {
  int real = BS;
  if (p.block_sizes) real = min(real, p.block_sizes[j]);
  real = min(real, p.Lkv - j * BS);
  return max(real, 0);
}

// Streams one [BS, D] bf16 tile (rows j*BS .. of head h) into swizzled LDS. One wave instruction
// moves 1 KiB = RPI rows; the XOR swizzle of a row only depends on the row's position within its
// instruction, so every lane keeps one source offset for the whole tile. Rows at or past `real`
// (the trailing partial block) re-read row 0 of the block: finite data that is masked (K) or
// multiplied by a zero probability (V), and nothing outside the tensor is touched.
template <int D, int BS, bool IS_V>
__device__ __forceinline__ int dma_lane_chunk(int w, int lane) {
  constexpr int CPR = D / 8;            // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;         // rows per wave instruction (4 or 8)
  const int rin = lane / CPR, pos = lane % CPR;
  const int sw = IS_V ? 2 * (rin & 3) : (rin + (RPI == 4 ? 4 * (w & 1) : 0)) & 7;
  return pos ^ sw;
}

template <int D, int BS>
__device__ __forceinline__ void dma_tile(bf16_t* lds, const bf16_t* tile, int64_t st, uint32_t lane_off,
                                         int chunk, int real, int w, int lane) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  constexpr int NW = BS / 32;
  constexpr int NI = BS / (RPI * NW);   // instructions per wave
  if (real >= BS) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r0 = (i * NW + w) * RPI;
      __builtin_amdgcn_global_load_lds((const void*)(tile + (int64_t)r0 * st + lane_off), WA_LDS(lds + r0 * D),
                                       16, 0, 0);
    }
  } else {
    const int rin = lane / CPR;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r0 = (i * NW + w) * RPI;
      const int row = r0 + rin;
      const bf16_t* g = tile + (int64_t)(row < real ? row : 0) * st + chunk * 8;
      __builtin_amdgcn_global_load_lds((const void*)g, WA_LDS(lds + r0 * D), 16, 0, 0);
    }
  }
}

template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) __attribute__((amdgpu_waves_per_eu(2)))
bsa_unit_kernel(FwdParams p) {
  constexpr int NW = BS / 32;
  constexpr int KT = BS / 32;   // 32-key tiles per key block
  constexpr int DC = D / 16;    // 16-wide chunks of the QK contraction
  constexpr int DT = D / 32;    // 32-wide output tiles of O^T
  constexpr int PC = BS / 16;   // 16-key chunks of the PV contraction
  constexpr int CPR = D / 8;
  constexpr int NI = D / 16;    // DMA instructions per wave per tile
  __shared__ __attribute__((aligned(1024))) bf16_t k_lds[BS * D];
  __shared__ __attribute__((aligned(1024))) bf16_t v_lds[BS * D];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;

  const int u = wa_xcd_remap(blockIdx.x, p.n_units);
  int64_t row;
  int split;
  if (p.units) {
    row = p.units[2 * u];
    split = p.units[2 * u + 1];
  } else {
    row = u / p.max_splits;
    split = u % p.max_splits;
  }
  if (row < 0 || row >= p.n_rows || split < 0 || split >= p.max_splits) return;
  const int qb = (int)(row % p.Nq);
  const int64_t bh = row / p.Nq;
  const int hs = (int)(bh % p.n_heads), b = (int)(bh / p.n_heads);
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;  // uniform per workgroup
  const int64_t irow = ((int64_t)b * p.H + h) * p.Nq + qb;

  const int n = row_visits(p, irow);
  const int s_begin = split * p.split;
  const int s_end = min(n, s_begin + p.split);
  if (s_begin >= s_end) return;  // unit beyond this row's list (an empty row is all zero)

  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  const bf16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;

  // Q^T fragments (B operand): lane holds Q[qi, 16c + 8g .. +8).
  bf16x8 qf[DC];
  {
    const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok ? qi : 0) * p.q_st;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      bf16x8 t = *(const bf16x8*)(qrow + c * 16 + g * 8);
      qf[c] = q_ok ? t : bf16x8{};
    }
  }

  // This unit's list entries, one per lane (split <= 64), read once: the loop below fetches them
  // with readlane and issues no memory reads besides the tile streams.
  const int cnt = s_end - s_begin;
  int my_j = 0, my_real = 0;
  if (lane < cnt) {
    my_j = p.index ? min(max(p.index[irow * p.index_width + s_begin + lane], 0), p.Nkv - 1) : s_begin + lane;
    my_real = block_real(p, my_j, BS);
  }
  uint64_t todo = __ballot(lane < cnt && my_real > 0);  // visits with at least one real key

  const int k_chunk = dma_lane_chunk<D, BS, false>(w, lane);
  const int v_chunk = dma_lane_chunk<D, BS, true>(w, lane);
  const uint32_t k_off = (uint32_t)((lane / CPR) * p.k_st + k_chunk * 8);
  const uint32_t v_off = (uint32_t)((lane / CPR) * p.v_st + v_chunk * 8);

  int j = 0, real = 0;
  if (todo) {
    const int cur = __builtin_ctzll(todo);
    todo &= todo - 1;
    j = __builtin_amdgcn_readlane(my_j, cur);
    real = __builtin_amdgcn_readlane(my_real, cur);
    dma_tile<D, BS>(k_lds, kbase + (int64_t)j * BS * p.k_st, p.k_st, k_off, k_chunk, real, w, lane);
    dma_tile<D, BS>(v_lds, vbase + (int64_t)j * BS * p.v_st, p.v_st, v_off, v_chunk, real, w, lane);
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
  float m_i = -INFINITY, l_i = 0.f;

  // Per-lane LDS read bases. K (A operand of S^T = K Q^T): lane reads row kt*32 + l32, chunk
  // 2c + g at position (2c + g) ^ (l32 & 7) = 8 (c / 4) + ((2 (c % 4) + g) ^ (l32 & 7)).
  const bf16_t* k_rd[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) k_rd[c] = k_lds + l32 * D + ((2 * c + g) ^ (l32 & 7)) * 8;
  // V (A operand of O^T += V^T P^T via transpose reads): 16-lane group G, source lane j = 4r + q
  // reads 4 elements of row 16c + 4(G/2) + 8hf + r at column 32t + 16(G%2) + 4q, whose chunk is
  // swizzled by 2r: 8 (t / 2) + ((4 (t % 2) + 2 (G % 2) + q / 2) ^ 2r).
  const int G = lane >> 4, tr_r = (lane & 15) >> 2, tr_q = lane & 3;
  const bf16_t* v_rd[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    v_rd[t] = v_lds + (4 * (G >> 1) + tr_r) * D + (((4 * t + 2 * (G & 1) + (tr_q >> 1)) ^ (2 * tr_r)) * 8) + 4 * (tr_q & 1);

  bool active = real > 0;
  while (active) {
    const int cur_real = real;
    const bool has_next = todo != 0;
    int j_next = 0, real_next = 0;
    if (has_next) {
      const int nxt = __builtin_ctzll(todo);
      todo &= todo - 1;
      j_next = __builtin_amdgcn_readlane(my_j, nxt);
      real_next = __builtin_amdgcn_readlane(my_real, nxt);
    }

    // ---- K tile ready (V of this tile may still stream) ----------------------------------
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NI) : "memory");

    f32x16 sacc[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) sacc[kt] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const bf16x8 a = *(const bf16x8*)(k_rd[c & 3] + (c >> 2) * 64 + kt * 32 * D);
        sacc[kt] = wa_mfma32(a, qf[c], sacc[kt]);
      }
    }
    wa_lds_barrier();  // every wave is done with K: stream the next K tile
    if (has_next)
      dma_tile<D, BS>(k_lds, kbase + (int64_t)j_next * BS * p.k_st, p.k_st, k_off, k_chunk, real_next, w, lane);

    // ---- online softmax in the log2 domain ------------------------------------------------
    float mx = -INFINITY;
    if (cur_real < BS) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= cur_real) sacc[kt][r] = -INFINITY;
        }
      }
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * p.scale_log2;
    const float m_new = fmaxf(m_i, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
    float rs = 0.f;
    bf16x8 pb[PC];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[kt][r], p.scale_log2, -m_new));
        rs += pv;
        pb[kt * 2 + (r >> 3)][r & 7] = (bf16_t)pv;
      }
    }
    l_i = fmaf(l_i, alpha, rs);
    m_i = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] *= alpha;

    // ---- V tile ready (the next K tile may still stream) -----------------------------------
    if (has_next) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int c = 0; c < PC; ++c) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        bf16x8 a;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const s16x4 vv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              WA_LDS4(v_rd[t & 1] + (16 * c + 8 * hf) * D + (t >> 1) * 64));
          const bf16x4 vb = __builtin_bit_cast(bf16x4, vv);
#pragma unroll
          for (int e = 0; e < 4; ++e) a[4 * hf + e] = vb[e];
        }
        oacc[t] = wa_mfma32(a, pb[c], oacc[t]);
      }
    }
    wa_lds_barrier();  // every wave is done with V: stream the next V tile
    if (has_next)
      dma_tile<D, BS>(v_lds, vbase + (int64_t)j_next * BS * p.v_st, p.v_st, v_off, v_chunk, real_next, w, lane);
    real = real_next;
    active = has_next;
  }

  // ---- normalized partial + log2-sum-exp -------------------------------------------------
  const float lsum = l_i + __shfl_xor(l_i, 32, 64);
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  const int64_t slot = row * p.max_splits + split;
  float* po = p.part_o + slot * (int64_t)(BS * D);
  const int ql = w * 32 + l32;
  if (g == 0) p.part_lse[slot * BS + ql] = lsum > 0.f ? m_i + log2f(lsum) : -INFINITY;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = t * 32 + 8 * rq + 4 * g;
      f32x4 ov = {oacc[t][rq * 4] * inv, oacc[t][rq * 4 + 1] * inv, oacc[t][rq * 4 + 2] * inv,
                  oacc[t][rq * 4 + 3] * inv};
      *(f32x4*)(po + ql * D + d0) = ov;
    }
  }
}

// Merges the partials of one row in split order, then the epilogue:
//   PLAIN: o = attn;  FUSE: o = attn + g * x;  GATED: o = g * attn,
// with g = sigmoid(q . gate_w[d] + gate_b[d]) (or sigmoid(q) without gate_w) — the gated fusion of
// attention.py:246-254 — and the natural-log LSE when asked for.
template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) bsa_combine_kernel(FwdParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int64_t row = blockIdx.x;
  const int qb = (int)(row % p.Nq);
  const int64_t bh = row / p.Nq;
  const int hs = (int)(bh % p.n_heads), b = (int)(bh / p.n_heads);
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  const int ql = w * 32 + l32;
  const int n = row_visits(p, ((int64_t)b * p.H + h) * p.Nq + qb);
  const int ns = min(n > 0 ? (n + p.split - 1) / p.split : 0, p.max_splits);
  const int64_t slot0 = row * p.max_splits;

  float M = -INFINITY;
  for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, p.part_lse[(slot0 + sp) * BS + ql]);
  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float Z = 0.f;
  if (M != -INFINITY) {
    for (int sp = 0; sp < ns; ++sp) {
      const float ls = p.part_lse[(slot0 + sp) * BS + ql];
      const float wgt = exp2f(ls - M);
      if (wgt == 0.f) continue;
      Z += wgt;
      const float* po = p.part_o + (slot0 + sp) * (int64_t)(BS * D) + ql * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 v = *(const f32x4*)(po + t * 32 + 8 * rq + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][rq * 4 + i] = fmaf(wgt, v[i], acc[t][rq * 4 + i]);
        }
      }
    }
  }
  const float inv = Z > 0.f ? 1.f / Z : 0.f;
  if (p.lse && g == 0 && q_ok)
    p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = Z > 0.f ? (M + log2f(Z)) * WA_LN2 : -INFINITY;

  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok ? qi : 0) * p.q_st;
  const bool need_gate = p.epilogue != WA_EPI_PLAIN;
  f32x16 gacc[DT];
  if (need_gate && p.gate_w) {
    bf16x8 qf[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      bf16x8 t = *(const bf16x8*)(qrow + c * 16 + g * 8);
      qf[c] = q_ok ? t : bf16x8{};
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      gacc[t] = f32x16{};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const bf16x8 a = *(const bf16x8*)(p.gate_w + (t * 32 + l32) * D + c * 16 + g * 8);
        gacc[t] = wa_mfma32(a, qf[c], gacc[t]);
      }
    }
  }
  if (!q_ok) return;

#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = t * 32 + 8 * rq + 4 * g;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = acc[t][rq * 4 + i] * inv;
        if (p.attn_round_bf16) a = wa_bf16_round(a);
        val[i] = a;
      }
      if (need_gate) {
        float gv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float pre;
          if (p.gate_w) {
            pre = gacc[t][rq * 4 + i] + (p.gate_b ? p.gate_b[d0 + i] : 0.f);
          } else {
            pre = (float)qrow[d0 + i];
          }
          if (p.gate_pre_bf16) pre = wa_bf16_round(pre);
          float gs = wa_sigmoid(pre);
          if (p.gate_out_bf16) gs = wa_bf16_round(gs);
          gv[i] = gs;
        }
        if (p.epilogue == WA_EPI_FUSE) {
          const int64_t xo = (int64_t)b * p.x_sb + (int64_t)qi * p.x_st + (int64_t)h * p.x_sh + d0;
#pragma unroll
          for (int i = 0; i < 4; ++i) val[i] = __fadd_rn(val[i], __fmul_rn(wa_load_f(p.x, xo + i, p.x_dtype), gv[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) val[i] = __fmul_rn(val[i], gv[i]);
        }
      }
      const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh + d0;
      if (p.o_dtype == WA_BF16) {
        bf16x4 ov = {(bf16_t)val[0], (bf16_t)val[1], (bf16_t)val[2], (bf16_t)val[3]};
        *(bf16x4*)((bf16_t*)p.o + oo) = ov;
      } else {
        f32x4 ov = {val[0], val[1], val[2], val[3]};
        *(f32x4*)((float*)p.o + oo) = ov;
      }
    }
  }
}

template <int D, int BS>
int launch(const FwdParams& fp, int64_t rows, hipStream_t stream) {
  hipLaunchKernelGGL((bsa_unit_kernel<D, BS>), dim3(fp.n_units), dim3(2 * BS), 0, stream, fp);
  int rc = wa_launch_status("bsa_fwd_unit");
  if (rc != WA_OK) return rc;
  hipLaunchKernelGGL((bsa_combine_kernel<D, BS>), dim3((unsigned)rows), dim3(2 * BS), 0, stream, fp);
  return wa_launch_status("bsa_fwd_combine");
}

int64_t split_slots(int64_t rows, int64_t max_visits, int64_t split) {
  const int64_t ms = max_visits > 0 ? (max_visits + split - 1) / split : 1;
  return rows * ms;
}

}  // namespace

extern "C" int64_t wa_bsa_fwd_workspace_bytes(int64_t rows, int64_t max_visits, int64_t split, int64_t block_size,
                                              int64_t D) {
  if (split <= 0) split = WA_BSA_DEFAULT_SPLIT;
  const int64_t slots = split_slots(rows, max_visits, split);
  return ((slots * block_size * (D + 1)) * 4 + 255) / 256 * 256;
}

extern "C" int wa_bsa_fwd(const wa_bsa_fwd_args* a, void* stream) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_fwd: null args");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_bsa_fwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_bsa_fwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0, "wa_bsa_fwd: bad sizes");
  WA_CHECK_ARG(a->q && a->k && a->v && a->o, "wa_bsa_fwd: null tensor");
  WA_CHECK_ARG(a->workspace, "wa_bsa_fwd: workspace required (wa_bsa_fwd_workspace_bytes)");
  WA_CHECK_ARG(wa_aligned16(a->q) && wa_aligned16(a->k) && wa_aligned16(a->v) && wa_aligned16(a->workspace),
               "wa_bsa_fwd: q/k/v/workspace must be 16-byte aligned");
  WA_CHECK_ARG(a->q_sb % 8 == 0 && a->q_st % 8 == 0 && a->q_sh % 8 == 0 && a->k_sb % 8 == 0 &&
                   a->k_st % 8 == 0 && a->k_sh % 8 == 0 && a->v_sb % 8 == 0 && a->v_st % 8 == 0 &&
                   a->v_sh % 8 == 0,
               "wa_bsa_fwd: q/k/v strides must be multiples of 8 elements");
  WA_CHECK_ARG(a->o_dtype == WA_F32 || a->o_dtype == WA_BF16, "wa_bsa_fwd: bad output dtype");
  const uintptr_t oal = a->o_dtype == WA_F32 ? 15u : 7u;
  WA_CHECK_ARG((((uintptr_t)a->o) & oal) == 0 && a->o_sb % 4 == 0 && a->o_st % 4 == 0 && a->o_sh % 4 == 0,
               "wa_bsa_fwd: output must be 4-element aligned with strides multiple of 4");
  WA_CHECK_ARG(a->epilogue >= WA_EPI_PLAIN && a->epilogue <= WA_EPI_GATED, "wa_bsa_fwd: bad epilogue");
  if (a->epilogue == WA_EPI_FUSE)
    WA_CHECK_ARG(a->x && (a->x_dtype == WA_F32 || a->x_dtype == WA_BF16), "wa_bsa_fwd: FUSE needs x");
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "wa_bsa_fwd: gate_w must be 16-byte aligned");
  if (a->index) WA_CHECK_ARG(a->num && a->index_width > 0, "wa_bsa_fwd: index needs num and width");
  const int64_t nq = (a->Lq + a->block_size - 1) / a->block_size;
  const int64_t nkv = (a->Lkv + a->block_size - 1) / a->block_size;
  const int64_t nh = a->heads ? a->n_heads : a->H;
  WA_CHECK_ARG(nh >= 0 && nh <= a->H, "wa_bsa_fwd: bad head count");
  const int64_t rows = a->B * nh * nq;
  const int64_t split = a->split_visits > 0 ? a->split_visits : WA_BSA_DEFAULT_SPLIT;
  WA_CHECK_ARG(split <= 64, "wa_bsa_fwd: split_visits %lld exceeds 64", (long long)split);
  const int64_t width = a->index ? a->index_width : nkv;
  const int64_t max_visits = a->max_visits > 0 ? (a->max_visits < width ? a->max_visits : width) : width;
  const int64_t max_splits = max_visits > 0 ? (max_visits + split - 1) / split : 1;
  const int64_t n_units = a->units ? a->n_units : rows * max_splits;
  WA_CHECK_ARG(rows < (int64_t)1 << 31 && n_units < (int64_t)1 << 31 && rows * max_splits < (int64_t)1 << 40 &&
                   a->Lq < (int64_t)1 << 30 && a->Lkv < (int64_t)1 << 30,
               "wa_bsa_fwd: problem too large");
  WA_CHECK_ARG(a->units == nullptr || a->n_units >= 0, "wa_bsa_fwd: bad unit count");
  if (rows == 0) return WA_OK;

  FwdParams fp{};
  fp.q = (const bf16_t*)a->q; fp.q_sb = a->q_sb; fp.q_st = a->q_st; fp.q_sh = a->q_sh;
  fp.k = (const bf16_t*)a->k; fp.k_sb = a->k_sb; fp.k_st = a->k_st; fp.k_sh = a->k_sh;
  fp.v = (const bf16_t*)a->v; fp.v_sb = a->v_sb; fp.v_st = a->v_st; fp.v_sh = a->v_sh;
  fp.o = a->o; fp.o_sb = a->o_sb; fp.o_st = a->o_st; fp.o_sh = a->o_sh; fp.o_dtype = a->o_dtype;
  fp.lse = a->lse;
  fp.index = a->index; fp.num = a->num; fp.index_width = a->index_width;
  fp.block_sizes = a->block_sizes;
  fp.heads = a->heads; fp.n_heads = (int)nh;
  fp.B = (int)a->B; fp.H = (int)a->H; fp.Lq = (int)a->Lq; fp.Lkv = (int)a->Lkv;
  fp.Nq = (int)nq; fp.Nkv = (int)nkv;
  const float scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->D);
  fp.scale_log2 = scale * WA_LOG2E;
  fp.epilogue = a->epilogue;
  fp.x = a->x; fp.x_sb = a->x_sb; fp.x_st = a->x_st; fp.x_sh = a->x_sh; fp.x_dtype = a->x_dtype;
  fp.gate_w = (const bf16_t*)a->gate_w; fp.gate_b = a->gate_b;
  fp.gate_pre_bf16 = a->gate_pre_bf16; fp.gate_out_bf16 = a->gate_out_bf16;
  fp.attn_round_bf16 = a->attn_round_bf16;
  fp.units = a->units; fp.n_units = (int)n_units; fp.max_splits = (int)max_splits; fp.split = (int)split;
  fp.n_rows = rows;
  fp.part_o = (float*)a->workspace;
  fp.part_lse = fp.part_o + rows * max_splits * a->block_size * a->D;
  if (n_units == 0) fp.n_units = 0;

  hipStream_t s = (hipStream_t)stream;
  if (fp.n_units == 0) {
    // nothing to visit: the combine pass still writes the (empty-row) outputs
    hipLaunchKernelGGL((a->D == 64 ? (a->block_size == 64 ? bsa_combine_kernel<64, 64> : bsa_combine_kernel<64, 128>)
                                   : (a->block_size == 64 ? bsa_combine_kernel<128, 64> : bsa_combine_kernel<128, 128>)),
                       dim3((unsigned)rows), dim3(2 * a->block_size), 0, s, fp);
    return wa_launch_status("bsa_fwd_combine");
  }
  if (a->D == 64 && a->block_size == 64) return launch<64, 64>(fp, rows, s);
  if (a->D == 64 && a->block_size == 128) return launch<64, 128>(fp, rows, s);
  if (a->D == 128 && a->block_size == 64) return launch<128, 64>(fp, rows, s);
  return launch<128, 128>(fp, rows, s);
}
