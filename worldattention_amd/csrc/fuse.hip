// Gated fusion of the two HSA branches as separate kernels (the training path; inference fuses it
// into the epilogue of whichever kernel writes a head last). Reference: attention.py:246-254,
//   gate = sigmoid(gate_lin(q)),  out = sparse + gate * linear,
// extended per head by the north-star head modes: sparse-only heads output `sparse`,
// linear-only heads `gate * linear`.
//
// fwd: one workgroup per (32-token tile (64 at D = 64), head, batch), one 32-channel tile per
//      wave; the gate pre-activation G^T = W Q^T is one MFMA product per wave (accumulator layout:
//      lane = token, registers = channels), the same arithmetic as the inference epilogue.
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
  int bias_vec;  // gate_b is 16-byte aligned (4-channel vector loads)
  int dout_vec;  // dout rows allow 4-channel vector loads
  int dq_vec;    // dq is 16-byte aligned with 16-byte aligned rows
  int B, H, L;
  // backward
  const void* dout; int64_t d_sb, d_st, d_sh; int d_dtype;
  float* dlin; int64_t dl_sb, dl_st, dl_sh;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int dq_acc;
  float* part;  // [n_tiles][B][H][D*D + D]
  float* dw; float* db;
  int n_tiles;
};

// fwd: workgroup = 32·(4 / DT) tokens of one (head, batch); wave w owns tokens 32·(w / DT).. and
// the 32-channel tile tt = w % DT, so a wave holds one tile of each operand (about 130 registers:
// three or four waves per SIMD) and the launch has enough small workgroups to stream.
template <int D>
__global__ void __launch_bounds__(256) fuse_fwd_kernel(FuseParams p) {
  constexpr int DC = D / 16, DT = D / 32, TG = 4 / DT;
  const int h = blockIdx.y, b = blockIdx.z;
  const int mode = p.modes[h];
  if (mode == 0) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int tt = w % DT;
  const int t = (blockIdx.x * TG + w / DT) * 32 + l32;
  const bool ok = t < p.L;
  const int64_t trow = ok ? t : 0;
  const int c0 = 32 * tt + 4 * g;  // this lane's channels: c0 + 8 rq + i (accumulator layout)
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + trow * p.q_st + (int64_t)h * p.q_sh;
  // Every read (sparse and linear outputs, q, the gate weight rows and bias) is issued before the
  // first store: on gfx9 loads and stores share one counter, so a load issued after a store waits
  // for that store.
  f32x4 sv[4], lv[4], pre_in[4];
  bf16x8 qf[DC], wf[DC];
  if (mode & MODE_SPARSE) {
    const float* src = p.sparse + (int64_t)b * p.s_sb + trow * p.s_st + (int64_t)h * p.s_sh + c0;
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) sv[rq] = *(const f32x4*)(src + 8 * rq);
  }
  if (mode & MODE_LINEAR) {
    const float* src = p.lin + (int64_t)b * p.l_sb + trow * p.l_st + (int64_t)h * p.l_sh + c0;
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) lv[rq] = *(const f32x4*)(src + 8 * rq);
    if (p.gate_w) {
      // G^T = W Q^T: A = rows 32 tt.. of W, B = the token's q (lane = token, registers = channels)
#pragma unroll
      for (int c = 0; c < DC; ++c) qf[c] = *(const bf16x8*)(qrow + c * 16 + g * 8);
#pragma unroll
      for (int c = 0; c < DC; ++c) wf[c] = *(const bf16x8*)(p.gate_w + (tt * 32 + l32) * D + c * 16 + g * 8);
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        if (!p.gate_b) {
          pre_in[rq] = f32x4{};
        } else if (p.bias_vec) {
          pre_in[rq] = *(const f32x4*)(p.gate_b + c0 + 8 * rq);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) pre_in[rq][i] = p.gate_b[c0 + 8 * rq + i];
        }
      }
    } else {  // sigmoid(q): the pre-activation is q itself
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const bf16x4 qv = *(const bf16x4*)(qrow + c0 + 8 * rq);
#pragma unroll
        for (int i = 0; i < 4; ++i) pre_in[rq][i] = (float)qv[i];
      }
    }
  }
  f32x16 gacc = f32x16{};
  if ((mode & MODE_LINEAR) && p.gate_w) {
#pragma unroll
    for (int c = 0; c < DC; ++c) gacc = wa_mfma32(wf[c], ok ? qf[c] : bf16x8{}, gacc);
  }
  if (!ok) return;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const int d0 = c0 + 8 * rq;
    float val[4] = {0.f, 0.f, 0.f, 0.f};
    if (mode & MODE_SPARSE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = p.attn_round_bf16 ? wa_bf16_round(sv[rq][i]) : sv[rq][i];
    }
    if (mode & MODE_LINEAR) {
      f32x4 gs;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float pre = p.gate_w ? gacc[rq * 4 + i] + pre_in[rq][i] : pre_in[rq][i];
        if (p.gate_pre_bf16) pre = wa_bf16_round(pre);
        float gv = wa_sigmoid(pre);
        if (p.gate_out_bf16) gv = wa_bf16_round(gv);
        gs[i] = gv;
        const float l = p.lin_round_bf16 ? wa_bf16_round(lv[rq][i]) : lv[rq][i];
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

// bwd: one workgroup of 8 waves per (128-token tile, linear head, batch), two waves per SIMD;
// wave w owns tokens 32 (w & 3).. and the channel half w >> 2 of every per-token pass.
template <int D>
__global__ void __launch_bounds__(512) fuse_bwd_kernel(FuseParams p) {
  constexpr int DC = D / 16, DT = D / 32, TTW = DT / 2;
  __shared__ __attribute__((aligned(1024))) bf16_t w_t[D * D];   // W [d][e]
  __shared__ __attribute__((aligned(1024))) bf16_t t_dg[128 * D];  // dgpre [token][d]
  __shared__ __attribute__((aligned(1024))) bf16_t t_q[128 * D];   // q [token][e]
  __shared__ float db_part[4][D];
  const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int mode = p.modes[h];
  if (!(mode & MODE_LINEAR)) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int half = w >> 2;
  if (p.gate_w) {
    for (int u = tid; u < D * D / 8; u += 512) tile_put8<D>(w_t, u / (D / 8), u % (D / 8), *(const bf16x8*)(p.gate_w + u * 8));
  }
  const int tl = (w & 3) * 32 + l32, t = tile * 128 + tl;
  const bool ok = t < p.L;
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(ok ? t : 0) * p.q_st + (int64_t)h * p.q_sh;
#pragma unroll
  for (int cc = 0; cc < DC / 2; ++cc) {
    const int c = half * (DC / 2) + cc;
    const bf16x8 v = *(const bf16x8*)(qrow + c * 16 + g * 8);
    tile_put8<D>(t_q, tl, 2 * c + g, ok ? v : bf16x8{});
  }
  // dgpre in accumulator layout (lane = token, channels d = 32 tt + 8 rq + 4 g + i). Per channel
  // tile all reads (lin, gate, dout, previous dq) are issued before any store, so they overlap
  // instead of waiting behind stores that might alias them.
  const int64_t lrow = (int64_t)b * p.l_sb + (int64_t)t * p.l_st + (int64_t)h * p.l_sh;
  const int64_t grow = (int64_t)b * p.g_sb + (int64_t)t * p.g_st + (int64_t)h * p.g_sh;
  const int64_t drow = (int64_t)b * p.d_sb + (int64_t)t * p.d_st + (int64_t)h * p.d_sh;
  const int64_t dlrow = (int64_t)b * p.dl_sb + (int64_t)t * p.dl_st + (int64_t)h * p.dl_sh;
  float* dq_row = p.dq + (int64_t)b * p.dq_sb + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
#pragma unroll
  for (int k = 0; k < TTW; ++k) {
    const int tt = half * TTW + k;
    f32x4 lv[4], gv[4], dy[4], prev[4];
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = 32 * tt + 8 * rq + 4 * g;
      if (ok) {
        lv[rq] = *(const f32x4*)(p.lin + lrow + d0);
        gv[rq] = *(const f32x4*)(p.gate + grow + d0);
        if (p.d_dtype == WA_BF16 && p.dout_vec) {
          const bf16x4 y = *(const bf16x4*)((const bf16_t*)p.dout + drow + d0);
#pragma unroll
          for (int i = 0; i < 4; ++i) dy[rq][i] = (float)y[i];
        } else if (p.dout_vec) {
          dy[rq] = *(const f32x4*)((const float*)p.dout + drow + d0);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            dy[rq][i] = p.d_dtype == WA_BF16 ? (float)((const bf16_t*)p.dout)[drow + d0 + i]
                                             : ((const float*)p.dout)[drow + d0 + i];
        }
        if (!p.gate_w && p.dq_acc) {
#pragma unroll
          for (int i = 0; i < 4; ++i) prev[rq][i] = dq_row[d0 + i];
        } else {
          prev[rq] = f32x4{};
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
      for (int i = 0; i < 4; ++i) d4[i] = (bf16_t)dg4[i];
      *(bf16x4*)(t_dg + tl * D + (((d0 >> 3) ^ dual_swizzle<D>(tl)) * 8) + (d0 & 7)) = d4;
    }
  }
  __syncthreads();
  if (!p.gate_w) return;
  // dq^T[e, t] += sum_d W[d, e] dgpre[t, d]: A = W^T by transpose reads, B = the token's dgpre row
#pragma unroll
  for (int k = 0; k < TTW; ++k) {
    const int et = half * TTW + k;
    f32x16 da = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) da = wa_mfma32(tile_tr8n<D>(w_t, c, 32 * et, lane), tile_row8<D>(t_dg, tl, 2 * c + g), da);
    if (ok) {
      // previous values read before any store
      float* dst = dq_row + 32 * et + 4 * g;
      f32x4 prev[4];
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        if (!p.dq_acc) {
          prev[rq] = f32x4{};
        } else if (p.dq_vec) {
          prev[rq] = *(const f32x4*)(dst + 8 * rq);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) prev[rq][i] = dst[8 * rq + i];
        }
      }
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = prev[rq][i] + da[rq * 4 + i];
        if (p.dq_vec) {
          *(f32x4*)(dst + 8 * rq) = o;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[8 * rq + i] = o[i];
        }
      }
    }
  }
  // partial dW[d, e] = sum_t dgpre[t, d] q[t, e] over this tile: DT x DT tiles of 32 x 32 spread
  // over the 8 waves; db[d] = sum_t dgpre[t, d] in four 32-token chains added in order
  float* part = p.part + (((int64_t)tile * p.B + b) * p.H + h) * (int64_t)(D * D + D);
  for (int i = w; i < DT * DT; i += 8) {
    const int dt = i / DT, et = i % DT;
    f32x16 pa = f32x16{};
#pragma unroll
    for (int c = 0; c < 8; ++c) pa = wa_mfma32(tile_tr8<D>(t_dg, c, 32 * dt, lane), tile_tr8<D>(t_q, c, 32 * et, lane), pa);
#pragma unroll
    for (int r = 0; r < 16; ++r) part[(32 * dt + 8 * (r >> 2) + 4 * g + (r & 3)) * D + 32 * et + l32] = pa[r];
  }
  if (tid < 4 * D) {
    const int d = tid % D, q4 = tid / D;
    float s = 0.f;
    for (int k = 0; k < 32; ++k) {
      const int tk = q4 * 32 + k;
      s += (float)t_dg[tk * D + (((d >> 3) ^ dual_swizzle<D>(tk)) * 8) + (d & 7)];
    }
    db_part[q4][d] = s;
  }
  __syncthreads();
  if (tid < D) part[D * D + tid] = ((db_part[0][tid] + db_part[1][tid]) + db_part[2][tid]) + db_part[3][tid];
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
  fp.bias_vec = a->gate_b && wa_aligned16(a->gate_b);
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
  const int64_t tokens_per_wg = a->D == 128 ? 32 : 64;
  dim3 grid((unsigned)((a->L + tokens_per_wg - 1) / tokens_per_wg), (unsigned)a->H, (unsigned)a->B);
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
  fp.dout_vec = (((uintptr_t)a->dout) & (a->dout_dtype == WA_F32 ? 15u : 7u)) == 0 && a->d_sb % 4 == 0 &&
                a->d_st % 4 == 0 && a->d_sh % 4 == 0;
  fp.dlin = a->dlin; fp.dl_sb = a->dl_sb; fp.dl_st = a->dl_st; fp.dl_sh = a->dl_sh;
  fp.dq = a->dq; fp.dq_sb = a->dq_sb; fp.dq_st = a->dq_st; fp.dq_sh = a->dq_sh; fp.dq_acc = a->dq_accumulate;
  fp.dq_vec = wa_aligned16(a->dq) && a->dq_sb % 4 == 0 && a->dq_st % 4 == 0 && a->dq_sh % 4 == 0;
  fp.part = (float*)a->workspace; fp.dw = a->dgate_w; fp.db = a->dgate_b;
  fp.n_tiles = (int)((a->L + 127) / 128);
  dim3 grid((unsigned)fp.n_tiles, (unsigned)a->H, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(fuse_bwd_kernel<128>, grid, dim3(512), 0, s, fp);
  else hipLaunchKernelGGL(fuse_bwd_kernel<64>, grid, dim3(512), 0, s, fp);
  if ((rc = wa_launch_status("hsa_fuse_bwd"))) return rc;
  if (a->gate_w) {
    const int64_t per = a->D * a->D + a->D;
    hipLaunchKernelGGL(fuse_reduce_kernel, dim3((unsigned)((per + FR_EL - 1) / FR_EL)), dim3(256), 0, s, fp, (int)a->D);
    return wa_launch_status("hsa_fuse_reduce");
  }
  return WA_OK;
}
