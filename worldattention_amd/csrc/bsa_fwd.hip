// Block-sparse flash-attention forward for gfx950 (bf16 MFMA 32x32x16, fp32 accumulation).
//
// One workgroup per (batch, head, query block); wave w owns query rows [32w, 32w+32) of the block.
// Per listed key block the workgroup stages K (row-major) and V (transposed) in LDS and every wave
// computes, with the transposed formulation
//     S^T[key, q] = K[key, :] . Q[q, :]        (A = K from LDS, B = Q^T from registers)
//     O^T[d, q]  += V^T[d, key] . P^T[key, q]  (A = V^T from LDS, B = P^T from registers)
// so that every lane owns one query column of S^T and O^T: row max / row sum need one exchange
// with lane^32, the rescale factor is a per-lane scalar, and the softmax probabilities feed the
// second MFMA directly from the first one's accumulator registers. The contraction order of the
// second product follows the accumulator layout; V^T is written to LDS with its keys permuted to
// the same order, so each A fragment is one 16-byte LDS read.
//
// Reference semantics: wan/modules/hsa/block_sparse_triton.py:67-139 (online softmax, partial
// trailing block mask, empty list -> 0) and block_sparse_torch.py:16-64 (id clamping, fp32 math).
#include "common.h"

namespace {

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
  int n_items;
};

// Position of key `kk` (0..BS-1) inside a transposed V row. The S^T accumulator register r of lane
// group g holds key 32*kt + 8*(r/4) + 4*g + r%4; the 16-key chunk c = 2*kt + r/8 is fed to the PV
// MFMA as the 8 registers r = 8*(c%2) .. +7 of each lane group, so chunk c occupies row positions
// [16c, 16c+16) with lane group g's 8 keys contiguous at 16c + 8g.
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk >> 4) * 16 + ((kk >> 2) & 1) * 8 + 4 * ((kk >> 3) & 1) + (kk & 3);
}

template <int D, int BS>
struct Stage {
  bf16x8 k[D / 16];
  bf16x8 v[D / 64][4];
};

template <int D, int BS>
__device__ __forceinline__ void load_tile(Stage<D, BS>& st, const FwdParams& p, int b, int h, int j,
                                          int real, int tid) {
  constexpr int NT = 2 * BS;
  constexpr int C8 = D / 8;
  const bf16_t* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + (int64_t)j * BS * p.k_st;
  const bf16_t* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + (int64_t)j * BS * p.v_st;
  const bf16x8 zero = {};
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int c = tid + i * NT, row = c / C8, col = (c % C8) * 8;
    st.k[i] = row < real ? *(const bf16x8*)(kb + (int64_t)row * p.k_st + col) : zero;
  }
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int u = tid + i * NT, key4 = u / C8, col = (u % C8) * 8;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = key4 * 4 + r;
      st.v[i][r] = row < real ? *(const bf16x8*)(vb + (int64_t)row * p.v_st + col) : zero;
    }
  }
}

template <int D, int BS>
__device__ __forceinline__ void store_tile(const Stage<D, BS>& st, bf16_t* k_lds, bf16_t* v_lds,
                                           int tid) {
  constexpr int NT = 2 * BS;
  constexpr int C8 = D / 8;
  constexpr int KLD = D + 8, VLD = BS + 8;
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const int c = tid + i * NT, row = c / C8, col = (c % C8) * 8;
    *(bf16x8*)(k_lds + row * KLD + col) = st.k[i];
  }
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int u = tid + i * NT, key4 = u / C8, col = (u % C8) * 8;
    const int pos = vt_pos(key4 * 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bf16x4 t = {st.v[i][0][e], st.v[i][1][e], st.v[i][2][e], st.v[i][3][e]};
      *(bf16x4*)(v_lds + (col + e) * VLD + pos) = t;
    }
  }
}

__device__ __forceinline__ int block_real(const FwdParams& p, int j, int BS) {
  int real = BS;
  if (p.block_sizes) real = min(real, p.block_sizes[j]);
  real = min(real, p.Lkv - j * BS);
  return max(real, 0);
}

template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) bsa_fwd_kernel(FwdParams p) {
  constexpr int KT = BS / 32;   // 32-key tiles per key block
  constexpr int DC = D / 16;    // 16-wide chunks of the QK contraction
  constexpr int DT = D / 32;    // 32-wide output tiles of O^T
  constexpr int PC = BS / 16;   // 16-key chunks of the PV contraction
  constexpr int KLD = D + 8, VLD = BS + 8;
  __shared__ __attribute__((aligned(16))) bf16_t k_lds[BS * KLD];
  __shared__ __attribute__((aligned(16))) bf16_t v_lds[D * VLD];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;

  const int item = wa_xcd_remap(blockIdx.x, p.n_items);
  const int qb = item % p.Nq;
  const int rest = item / p.Nq;
  const int hs = rest % p.n_heads, b = rest / p.n_heads;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;  // uniform per workgroup
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;

  // Q^T fragments (B operand): lane holds Q[qi, 16c + 8g .. +8).
  bf16x8 qf[DC];
  {
    const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)qi * p.q_st;
    const bf16x8 zero = {};
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = q_ok ? *(const bf16x8*)(qrow + c * 16 + g * 8) : zero;
  }

  const int64_t row = ((int64_t)b * p.H + h) * p.Nq + qb;
  int n;
  if (p.index) {
    n = p.num[row];
    n = max(0, min(n, (int)p.index_width));
  } else {
    n = p.Nkv;
  }
  const int32_t* list = p.index ? p.index + row * p.index_width : nullptr;
  auto block_id = [&](int s) -> int {
    return list ? min(max(list[s], 0), p.Nkv - 1) : s;
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
  float m_i = -INFINITY, l_i = 0.f;

  Stage<D, BS> st;
  int real_next = 0;
  if (n > 0) {
    const int j0 = block_id(0);
    real_next = block_real(p, j0, BS);
    load_tile<D, BS>(st, p, b, h, j0, real_next, tid);
  }

  for (int s = 0; s < n; ++s) {
    const int real = real_next;
    __syncthreads();
    store_tile<D, BS>(st, k_lds, v_lds, tid);
    __syncthreads();
    if (s + 1 < n) {
      const int jn = block_id(s + 1);
      real_next = block_real(p, jn, BS);
      load_tile<D, BS>(st, p, b, h, jn, real_next, tid);
    }

    // S^T = K Q^T
    f32x16 sacc[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      sacc[kt] = f32x16{};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const bf16x8 a = *(const bf16x8*)(k_lds + (kt * 32 + l32) * KLD + c * 16 + g * 8);
        sacc[kt] = wa_mfma32(a, qf[c], sacc[kt]);
      }
    }

    // online softmax in the log2 domain
    float mx = -INFINITY;
    const bool partial = real < BS;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = sacc[kt][r] * p.scale_log2;
        if (partial) {
          const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= real) x = -INFINITY;
        }
        sacc[kt][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_i, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_i - m_use);
    float rs = 0.f;
    bf16x8 pb[PC];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = exp2f(sacc[kt][r] - m_use);
        rs += pv;
        pb[kt * 2 + (r >> 3)][r & 7] = (bf16_t)pv;
      }
    }
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] *= alpha;

    // O^T += V^T P^T
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int c = 0; c < PC; ++c) {
        const bf16x8 a = *(const bf16x8*)(v_lds + (t * 32 + l32) * VLD + c * 16 + g * 8);
        oacc[t] = wa_mfma32(a, pb[c], oacc[t]);
      }
    }
  }

  const float lsum = l_i + __shfl_xor(l_i, 32, 64);
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  if (p.lse && g == 0 && q_ok)
    p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = lsum > 0.f ? (m_i + log2f(lsum)) * WA_LN2 : -INFINITY;

  // Gate G^T = W Q^T (same accumulator layout as O^T), only when the epilogue needs it.
  f32x16 gacc[DT];
  const bool need_gate = p.epilogue != WA_EPI_PLAIN;
  if (need_gate && p.gate_w) {
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

  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)qi * p.q_st;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = t * 32 + 8 * rq + 4 * g;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = oacc[t][rq * 4 + i] * inv;
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
int launch(const FwdParams& fp, hipStream_t stream) {
  hipLaunchKernelGGL((bsa_fwd_kernel<D, BS>), dim3(fp.n_items), dim3(2 * BS), 0, stream, fp);
  return wa_launch_status("bsa_fwd");
}

}  // namespace

extern "C" int wa_bsa_fwd(const wa_bsa_fwd_args* a, void* stream) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_fwd: null args");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_bsa_fwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_bsa_fwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0, "wa_bsa_fwd: bad sizes");
  WA_CHECK_ARG(a->q && a->k && a->v && a->o, "wa_bsa_fwd: null tensor");
  WA_CHECK_ARG(wa_aligned16(a->q) && wa_aligned16(a->k) && wa_aligned16(a->v),
               "wa_bsa_fwd: q/k/v must be 16-byte aligned");
  WA_CHECK_ARG(a->q_sb % 8 == 0 && a->q_st % 8 == 0 && a->q_sh % 8 == 0 && a->k_sb % 8 == 0 &&
                   a->k_st % 8 == 0 && a->k_sh % 8 == 0 && a->v_sb % 8 == 0 && a->v_st % 8 == 0 &&
                   a->v_sh % 8 == 0,
               "wa_bsa_fwd: q/k/v strides must be multiples of 8 elements");
  WA_CHECK_ARG(a->o_dtype == WA_F32 || a->o_dtype == WA_BF16, "wa_bsa_fwd: bad output dtype");
  WA_CHECK_ARG((((uintptr_t)a->o) & 7u) == 0 && a->o_sb % 4 == 0 && a->o_st % 4 == 0 && a->o_sh % 4 == 0,
               "wa_bsa_fwd: output must be 8-byte aligned with strides multiple of 4");
  WA_CHECK_ARG(a->epilogue >= WA_EPI_PLAIN && a->epilogue <= WA_EPI_GATED, "wa_bsa_fwd: bad epilogue");
  if (a->epilogue == WA_EPI_FUSE)
    WA_CHECK_ARG(a->x && (a->x_dtype == WA_F32 || a->x_dtype == WA_BF16), "wa_bsa_fwd: FUSE needs x");
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "wa_bsa_fwd: gate_w must be 16-byte aligned");
  if (a->index) WA_CHECK_ARG(a->num && a->index_width > 0, "wa_bsa_fwd: index needs num and width");
  const int64_t nq = (a->Lq + a->block_size - 1) / a->block_size;
  const int64_t nkv = (a->Lkv + a->block_size - 1) / a->block_size;
  const int64_t nh = a->heads ? a->n_heads : a->H;
  WA_CHECK_ARG(nh >= 0 && nh <= a->H, "wa_bsa_fwd: bad head count");
  const int64_t items = a->B * nh * nq;
  WA_CHECK_ARG(items < (int64_t)1 << 31 && a->Lq < (int64_t)1 << 30 && a->Lkv < (int64_t)1 << 30,
               "wa_bsa_fwd: problem too large");
  if (items == 0) return WA_OK;

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
  fp.n_items = (int)items;

  hipStream_t s = (hipStream_t)stream;
  if (a->D == 64 && a->block_size == 64) return launch<64, 64>(fp, s);
  if (a->D == 64 && a->block_size == 128) return launch<64, 128>(fp, s);
  if (a->D == 128 && a->block_size == 64) return launch<128, 64>(fp, s);
  return launch<128, 128>(fp, s);
}
