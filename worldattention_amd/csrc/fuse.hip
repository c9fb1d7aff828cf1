// Gated fusion of the two HSA branches as separate kernels (the training path; inference fuses it
// into the epilogue of whichever kernel writes a head last). Reference: attention.py:246-254,
//   gate = sigmoid(gate_lin(q)),  out = sparse + gate * linear,
// extended per head by the north-star head modes: sparse-only heads output `sparse`,
// linear-only heads `gate * linear`.
//
// fwd: one workgroup per (128-token tile, head, batch), wave w = tokens 32w..; the gate
//      pre-activation G^T = W Q^T is one MFMA product per wave (accumulator layout: lane = token,
//      registers = channels), the same arithmetic as the inference epilogue.
// bwd: dlinear = dout * g,  dgpre = dout * linear * g (1 - g),  dq += dgpre W (or dgpre when the
//      gate is sigmoid(q)), and per-tile partials of dW = dgpre^T q and db = sum dgpre, summed by
//      a second pass in a fixed order.
#include "tile.h"

namespace {

enum { MODE_SPARSE = 1, MODE_LINEAR = 2 };

struct FuseParams {
  const bf16_t* q; int64_t q_sb, q_st, q_sh;
  const float* sparse; int64_t s_sb, s_st, s_sh;
  const float* lin; int64_t l_sb, l_st, l_sh;
  const int32_t* modes;  // [H]
  void* out; int64_t o_sb, o_st, o_sh; int o_dtype;
  float* gate; int64_t g_sb, g_st, g_sh;
  const bf16_t* gate_w; const float* gate_b;
  int gate_pre_bf16, gate_out_bf16, attn_round_bf16, lin_round_bf16;
  int B, H, L;
  // backward
  const void* dout; int64_t d_sb, d_st, d_sh; int d_dtype;
  float* dlin; int64_t dl_sb, dl_st, dl_sh;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int dq_acc;
  float* part;  // [n_tiles][B][H][D*D + D]
  float* dw; float* db;
  int n_tiles;
};

template <int D>
__device__ __forceinline__ void gate_preact(const FuseParams& p, const bf16_t* qrow, bool ok, int g, int l32,
                                            f32x16 (&gacc)[D / 32], bf16x8 (&qf)[D / 16]) {
  constexpr int DC = D / 16, DT = D / 32;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    const bf16x8 t = *(const bf16x8*)(qrow + c * 16 + g * 8);
    qf[c] = ok ? t : bf16x8{};
  }
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    gacc[t] = f32x16{};
    if (p.gate_w) {
#pragma unroll
      for (int c = 0; c < DC; ++c)
        gacc[t] = wa_mfma32(*(const bf16x8*)(p.gate_w + (t * 32 + l32) * D + c * 16 + g * 8), qf[c], gacc[t]);
    }
  }
}


template <int D>
__global__ void __launch_bounds__(256) fuse_fwd_kernel(FuseParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int mode = p.modes[h];
  if (mode == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int t = tile * 128 + w * 32 + l32;
  const bool ok = t < p.L;
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(ok ? t : 0) * p.q_st + (int64_t)h * p.q_sh;
  // Every read of the row (sparse and linear outputs, q and the gate weights for the gate) is
  // issued before the first store: on gfx9 loads and stores share one counter, so a load issued
  // after a store waits for that store.
  const int64_t trow = ok ? t : 0;
  f32x4 sv[DT][4], lv[DT][4];
  if (mode & MODE_SPARSE) {
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        sv[tt][rq] = *(const f32x4*)(p.sparse + (int64_t)b * p.s_sb + trow * p.s_st + (int64_t)h * p.s_sh +
                                     32 * tt + 8 * rq + 4 * g);
  }
  if (mode & MODE_LINEAR) {
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        lv[tt][rq] = *(const f32x4*)(p.lin + (int64_t)b * p.l_sb + trow * p.l_st + (int64_t)h * p.l_sh +
                                     32 * tt + 8 * rq + 4 * g);
  }
  f32x16 gacc[DT];
  bf16x8 qf[DC];
  if (mode & MODE_LINEAR) gate_preact<D>(p, qrow, ok, g, l32, gacc, qf);
  float pre_in[DT][4][4];  // gate bias, or q itself for the sigmoid(q) gate, before any store
  if (mode & MODE_LINEAR) {
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * tt + 8 * rq + 4 * g + i;
          pre_in[tt][rq][i] = p.gate_w ? (p.gate_b ? p.gate_b[d] : 0.f) : (float)qrow[d];
        }
  }
  if (!ok) return;
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * tt + 8 * rq + 4 * g;
      float val[4] = {0.f, 0.f, 0.f, 0.f};
      if (mode & MODE_SPARSE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) val[i] = p.attn_round_bf16 ? wa_bf16_round(sv[tt][rq][i]) : sv[tt][rq][i];
      }
      if (mode & MODE_LINEAR) {
        f32x4 gs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float pre = p.gate_w ? gacc[tt][rq * 4 + i] + pre_in[tt][rq][i] : pre_in[tt][rq][i];
          if (p.gate_pre_bf16) pre = wa_bf16_round(pre);
          float gv = wa_sigmoid(pre);
          if (p.gate_out_bf16) gv = wa_bf16_round(gv);
          gs[i] = gv;
          const float l = p.lin_round_bf16 ? wa_bf16_round(lv[tt][rq][i]) : lv[tt][rq][i];
          val[i] = (mode & MODE_SPARSE) ? wa_add_rn(val[i], wa_mul_rn(l, gs[i])) : wa_mul_rn(l, gs[i]);
        }
        if (p.gate) *(f32x4*)(p.gate + (int64_t)b * p.g_sb + (int64_t)t * p.g_st + (int64_t)h * p.g_sh + d0) = gs;
      }
      const int64_t oo = (int64_t)b * p.o_sb + (int64_t)t * p.o_st + (int64_t)h * p.o_sh + d0;
      if (p.o_dtype == WA_BF16) {
        bf16x4 ov = {(bf16_t)val[0], (bf16_t)val[1], (bf16_t)val[2], (bf16_t)val[3]};
        *(bf16x4*)((bf16_t*)p.out + oo) = ov;
      } else {
        f32x4 ov = {val[0], val[1], val[2], val[3]};
        *(f32x4*)((float*)p.out + oo) = ov;
      }
    }
  }
}

template <int D>
__global__ void __launch_bounds__(256) fuse_bwd_kernel(FuseParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(1024))) bf16_t w_t[D * D];   // W [d][e]
  __shared__ __attribute__((aligned(1024))) bf16_t t_dg[128 * D];  // dgpre [token][d]
  __shared__ __attribute__((aligned(1024))) bf16_t t_q[128 * D];   // q [token][e]
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int mode = p.modes[h];
  if (!(mode & MODE_LINEAR)) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  if (p.gate_w) {
    for (int u = tid; u < D * D / 8; u += 256) tile_put8<D>(w_t, u / (D / 8), u % (D / 8), *(const bf16x8*)(p.gate_w + u * 8));
  }
  const int tl = w * 32 + l32, t = tile * 128 + tl;
  const bool ok = t < p.L;
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(ok ? t : 0) * p.q_st + (int64_t)h * p.q_sh;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    const bf16x8 v = *(const bf16x8*)(qrow + c * 16 + g * 8);
    tile_put8<D>(t_q, tl, 2 * c + g, ok ? v : bf16x8{});
  }
  // dgpre in accumulator layout (lane = token, channels d = 32 tt + 8 (r / 4) + 4 g + r % 4).
  // Per channel tile all reads (lin, gate, dout, previous dq) are issued before any store, so
  // they overlap instead of waiting behind stores that might alias them.
  bf16x8 dgb[DC];
  const int64_t lrow = (int64_t)b * p.l_sb + (int64_t)t * p.l_st + (int64_t)h * p.l_sh;
  const int64_t grow = (int64_t)b * p.g_sb + (int64_t)t * p.g_st + (int64_t)h * p.g_sh;
  const int64_t drow = (int64_t)b * p.d_sb + (int64_t)t * p.d_st + (int64_t)h * p.d_sh;
  const int64_t dlrow = (int64_t)b * p.dl_sb + (int64_t)t * p.dl_st + (int64_t)h * p.dl_sh;
  float* dq_row = p.dq + (int64_t)b * p.dq_sb + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
#pragma unroll
  for (int tt = 0; tt < DT; ++tt) {
    f32x4 lv[4], gv[4];
    float dy[4][4], prev[4][4];
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * tt + 8 * rq + 4 * g;
      if (ok) {
        lv[rq] = *(const f32x4*)(p.lin + lrow + d0);
        gv[rq] = *(const f32x4*)(p.gate + grow + d0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dy[rq][i] = p.d_dtype == WA_BF16 ? (float)((const bf16_t*)p.dout)[drow + d0 + i]
                                           : ((const float*)p.dout)[drow + d0 + i];
          prev[rq][i] = !p.gate_w && p.dq_acc ? dq_row[d0 + i] : 0.f;
        }
      }
    }
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * tt + 8 * rq + 4 * g;
      float dg4[4] = {0.f, 0.f, 0.f, 0.f};
      if (ok) {
        f32x4 dl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float l = p.lin_round_bf16 ? wa_bf16_round(lv[rq][i]) : lv[rq][i];
          dl[i] = dy[rq][i] * gv[rq][i];
          dg4[i] = dy[rq][i] * l * gv[rq][i] * (1.f - gv[rq][i]);
        }
        *(f32x4*)(p.dlin + dlrow + d0) = dl;
        if (!p.gate_w) {
#pragma unroll
          for (int i = 0; i < 4; ++i) dq_row[d0 + i] = prev[rq][i] + dg4[i];
        }
      }
      bf16x4 d4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dgb[2 * tt + (rq >> 1)][(rq & 1) * 4 + i] = (bf16_t)dg4[i];
        d4[i] = (bf16_t)dg4[i];
      }
      *(bf16x4*)(t_dg + tl * D + (((d0 >> 3) ^ dual_swizzle<D>(tl)) * 8) + (d0 & 7)) = d4;
    }
  }
  __syncthreads();
  if (!p.gate_w) return;
  // dq^T[e, t] += sum_d W[d, e] dgpre[t, d]: A = W^T by transpose reads in accumulator order
#pragma unroll
  for (int et = 0; et < DT; ++et) {
    f32x16 da = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) da = wa_mfma32(tile_tr8<D>(w_t, c, 32 * et, lane), dgb[c], da);
    if (ok) {
      // previous values read before any store
      float* dst = p.dq + (int64_t)b * p.dq_sb + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
      float prev[4][4];
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
#pragma unroll
        for (int i = 0; i < 4; ++i) prev[rq][i] = p.dq_acc ? dst[32 * et + 8 * rq + 4 * g + i] : 0.f;
      }
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[32 * et + 8 * rq + 4 * g + i] = prev[rq][i] + da[rq * 4 + i];
      }
    }
  }
  // partial dW[d, e] = sum_t dgpre[t, d] q[t, e] and db[d] = sum_t dgpre[t, d] over this tile
  float* part = p.part + (((int64_t)tile * p.B + b) * p.H + h) * (int64_t)(D * D + D);
  constexpr int TPW = DT * DT / 4;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int dt = D == 128 ? w : (w >> 1);
    const int et = D == 128 ? i : (w & 1);
    f32x16 pa = f32x16{};
#pragma unroll
    for (int c = 0; c < 8; ++c) pa = wa_mfma32(tile_tr8<D>(t_dg, c, 32 * dt, lane), tile_tr8<D>(t_q, c, 32 * et, lane), pa);
#pragma unroll
    for (int r = 0; r < 16; ++r) part[(32 * dt + 8 * (r >> 2) + 4 * g + (r & 3)) * D + 32 * et + l32] = pa[r];
  }
  for (int d = tid; d < D; d += 256) {
    float s = 0.f;
    for (int tt = 0; tt < 128; ++tt) s += (float)t_dg[tt * D + (((d >> 3) ^ dual_swizzle<D>(tt)) * 8) + (d & 7)];
    part[D * D + d] = s;
  }
}

// dW, db: sum of the per-(tile, batch, linear head) partials in a fixed order (bitwise
// reproducible). A workgroup covers 32 consecutive elements (one 128-byte line of every partial)
// with 8 groups of 32 threads; group g sums the linear-head partials g, g + 8, ... (in the order
// tile, batch, linear head) in eight chains with eight loads in flight, and the group sums are
// added in group order. Partials of heads without a linear branch are never read.
constexpr int FR_EL = 32, FR_G = 8, FR_MAX_H = 256;
__global__ void __launch_bounds__(256) fuse_reduce_kernel(FuseParams p, int D) {
  __shared__ float red[FR_G][FR_EL];
  __shared__ int s_lin[FR_MAX_H];
  __shared__ int s_nlin;
  if (threadIdx.x == 0) {
    int n = 0;
    for (int h = 0; h < p.H; ++h)
      if (p.modes[h] & MODE_LINEAR) s_lin[n++] = h;
    s_nlin = n;
  }
  __syncthreads();
  const int64_t per = (int64_t)D * D + D;
  const int el = threadIdx.x % FR_EL, grp = threadIdx.x / FR_EL;
  const int64_t i = (int64_t)blockIdx.x * FR_EL + el;
  const int nlin = s_nlin, n_src = p.n_tiles * p.B * nlin;
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = 0.f;
  if (i < per) {
    const float* col = p.part + i;
    for (int k0 = grp; k0 < n_src; k0 += 8 * FR_G) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = k0 + q * FR_G;
        const int tb = k / max(nlin, 1);  // (tile * B + b)
        v[q] = k < n_src ? col[((int64_t)tb * p.H + s_lin[k - tb * nlin]) * per] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) a[q] += v[q];
    }
  }
  red[grp][el] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  __syncthreads();
  if (grp == 0 && i < per) {
    float s = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < FR_G; ++g2) s += red[g2][el];
    if (i < (int64_t)D * D) p.dw[i] = s;
    else p.db[i - (int64_t)D * D] = s;
  }
}

void fill_common(FuseParams& fp, const wa_hsa_fuse_args* a) {
  fp.q = (const bf16_t*)a->q; fp.q_sb = a->q_sb; fp.q_st = a->q_st; fp.q_sh = a->q_sh;
  fp.sparse = a->sparse; fp.s_sb = a->s_sb; fp.s_st = a->s_st; fp.s_sh = a->s_sh;
  fp.lin = a->lin; fp.l_sb = a->l_sb; fp.l_st = a->l_st; fp.l_sh = a->l_sh;
  fp.modes = a->head_modes;
  fp.gate = a->gate; fp.g_sb = a->g_sb; fp.g_st = a->g_st; fp.g_sh = a->g_sh;
  fp.gate_w = (const bf16_t*)a->gate_w; fp.gate_b = a->gate_b;
  fp.gate_pre_bf16 = a->gate_pre_bf16; fp.gate_out_bf16 = a->gate_out_bf16;
  fp.attn_round_bf16 = a->attn_round_bf16; fp.lin_round_bf16 = a->lin_round_bf16;
  fp.B = (int)a->B; fp.H = (int)a->H; fp.L = (int)a->L;
}

int check_common(const wa_hsa_fuse_args* a, const char* who) {
  WA_CHECK_ARG(a && a->q && a->head_modes, "%s: null argument", who);
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "%s: head dim %lld not in {64, 128}", who, (long long)a->D);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->L >= 0, "%s: bad sizes", who);
  WA_CHECK_ARG(wa_aligned16(a->q) && a->q_sb % 8 == 0 && a->q_st % 8 == 0 && a->q_sh % 8 == 0,
               "%s: q must be 16-byte aligned with 16-byte aligned rows", who);
  if (a->sparse) WA_CHECK_ARG(wa_aligned16(a->sparse) && a->s_sb % 4 == 0 && a->s_st % 4 == 0 && a->s_sh % 4 == 0, "%s: sparse alignment", who);
  if (a->lin) WA_CHECK_ARG(wa_aligned16(a->lin) && a->l_sb % 4 == 0 && a->l_st % 4 == 0 && a->l_sh % 4 == 0, "%s: lin alignment", who);
  if (a->gate) WA_CHECK_ARG(wa_aligned16(a->gate) && a->g_sb % 4 == 0 && a->g_st % 4 == 0 && a->g_sh % 4 == 0, "%s: gate alignment", who);
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "%s: gate_w must be 16-byte aligned", who);
  return WA_OK;
}

}  // namespace

extern "C" int wa_hsa_fuse_fwd(const wa_hsa_fuse_args* a, void* stream) {
  int rc = check_common(a, "wa_hsa_fuse_fwd");
  if (rc) return rc;
  WA_CHECK_ARG(a->out && (a->o_dtype == WA_F32 || a->o_dtype == WA_BF16), "wa_hsa_fuse_fwd: bad output");
  WA_CHECK_ARG((((uintptr_t)a->out) & (a->o_dtype == WA_F32 ? 15u : 7u)) == 0 && a->o_sb % 4 == 0 && a->o_st % 4 == 0 &&
                   a->o_sh % 4 == 0,
               "wa_hsa_fuse_fwd: output alignment");
  if (a->B == 0 || a->L == 0) return WA_OK;
  FuseParams fp{};
  fill_common(fp, a);
  fp.out = a->out; fp.o_sb = a->o_sb; fp.o_st = a->o_st; fp.o_sh = a->o_sh; fp.o_dtype = a->o_dtype;
  dim3 grid((unsigned)((a->L + 127) / 128), (unsigned)a->H, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(fuse_fwd_kernel<128>, grid, dim3(256), 0, s, fp);
  else hipLaunchKernelGGL(fuse_fwd_kernel<64>, grid, dim3(256), 0, s, fp);
  return wa_launch_status("hsa_fuse_fwd");
}

extern "C" int64_t wa_hsa_fuse_bwd_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t D) {
  const int64_t tiles = (L + 127) / 128;
  return ((tiles * B * H * (D * D + D)) * 4 + 255) / 256 * 256;
}

extern "C" int wa_hsa_fuse_bwd(const wa_hsa_fuse_args* a, void* stream) {
  int rc = check_common(a, "wa_hsa_fuse_bwd");
  if (rc) return rc;
  WA_CHECK_ARG(a->dout && a->lin && a->gate && a->dlin && a->dq, "wa_hsa_fuse_bwd: dout, lin, gate, dlin, dq required");
  WA_CHECK_ARG(a->dout_dtype == WA_F32 || a->dout_dtype == WA_BF16, "wa_hsa_fuse_bwd: bad dout dtype");
  WA_CHECK_ARG(wa_aligned16(a->dlin) && a->dl_sb % 4 == 0 && a->dl_st % 4 == 0 && a->dl_sh % 4 == 0,
               "wa_hsa_fuse_bwd: dlin alignment");
  if (a->gate_w) WA_CHECK_ARG(a->workspace && a->dgate_w && a->dgate_b, "wa_hsa_fuse_bwd: gate_w needs workspace, dgate_w, dgate_b");
  WA_CHECK_ARG(a->H <= FR_MAX_H, "wa_hsa_fuse_bwd: at most %d heads", FR_MAX_H);
  if (a->B == 0 || a->L == 0) return WA_OK;
  FuseParams fp{};
  fill_common(fp, a);
  fp.dout = a->dout; fp.d_sb = a->d_sb; fp.d_st = a->d_st; fp.d_sh = a->d_sh; fp.d_dtype = a->dout_dtype;
  fp.dlin = a->dlin; fp.dl_sb = a->dl_sb; fp.dl_st = a->dl_st; fp.dl_sh = a->dl_sh;
  fp.dq = a->dq; fp.dq_sb = a->dq_sb; fp.dq_st = a->dq_st; fp.dq_sh = a->dq_sh; fp.dq_acc = a->dq_accumulate;
  fp.part = (float*)a->workspace; fp.dw = a->dgate_w; fp.db = a->dgate_b;
  fp.n_tiles = (int)((a->L + 127) / 128);
  dim3 grid((unsigned)fp.n_tiles, (unsigned)a->H, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(fuse_bwd_kernel<128>, grid, dim3(256), 0, s, fp);
  else hipLaunchKernelGGL(fuse_bwd_kernel<64>, grid, dim3(256), 0, s, fp);
  if ((rc = wa_launch_status("hsa_fuse_bwd"))) return rc;
  if (a->gate_w) {
    const int64_t per = a->D * a->D + a->D;
    hipLaunchKernelGGL(fuse_reduce_kernel, dim3((unsigned)((per + FR_EL - 1) / FR_EL)), dim3(256), 0, s, fp, (int)a->D);
    return wa_launch_status("hsa_fuse_reduce");
  }
  return WA_OK;
}
