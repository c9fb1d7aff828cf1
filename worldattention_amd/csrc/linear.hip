// Linear-branch kernels for gfx950:
//  * compress_kv  — low-rank sequence projection per segment (attention.py:64-110);
//  * elu1 state   — S^T = V^T phi(K), z = sum phi(K) over the KV window (north-star linear heads);
//  * elu1 readout — o = phi(q) S / (phi(q) . z), with the gated-fusion epilogue.
// All contractions run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation. Operands whose
// contraction index is the token axis are staged through LDS transposed ([channel][token]).
#include "common.h"

namespace {

__device__ __forceinline__ float elu1f(float x) { return x > 0.f ? x + 1.f : __expf(x); }

template <typename T>
__device__ __forceinline__ void load8(const T* src, float (&f)[8], bool ok) {
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = ok ? (float)src[e] : 0.f;
}

// =============================================================================================
// compress_kv: out[row0 + r, d] = sum_t E[r, t] x[start + t, d], one workgroup per
// (segment, head, batch). Tokens are processed 64 at a time: x^T chunk in LDS, E fragments read
// from global (tiny, cache resident). Wave w owns output column tiles w, w+4, ...
// =============================================================================================
struct CompressParams {
  const void* x; int64_t x_sb, x_st, x_sh; int x_dtype;
  const void* proj; int proj_dtype; int proj_rank, proj_len;
  int L, H, D, seg, block;
  void* out; int64_t o_sb, o_st, o_sh; int o_dtype;
};

template <int D>
__global__ void __launch_bounds__(256) compress_kernel(CompressParams p) {
  constexpr int TC = 64;              // tokens per LDS chunk
  constexpr int XLD = TC + 8;
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(16))) bf16_t xt[D * XLD];
  const int sidx = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int start = sidx * p.seg;
  const int seg_len = min(p.seg, p.L - start);
  const int rank = min(p.proj_rank, (seg_len + p.block - 1) / p.block);
  const int row0 = sidx * min(p.proj_rank, (p.seg + p.block - 1) / p.block);
  const int mtiles = (rank + 31) / 32;

  // wave w owns output column tile w (D <= 128, so at most one tile per wave)
  const bool wave_active = w < DT;
  f32x16 acc[4];  // [m tile]
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m] = f32x16{};

  for (int t0 = 0; t0 < seg_len; t0 += TC) {
    __syncthreads();
    // stage x[start+t0 .. +TC, :] transposed: unit = 4 tokens x 8 channels
    for (int u = tid; u < (TC / 4) * (D / 8); u += 256) {
      const int tq = u / (D / 8), c8 = (u % (D / 8)) * 8;
      float f[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + tq * 4 + r;
        const bool ok = t < seg_len;
        const int64_t off = (int64_t)b * p.x_sb + (int64_t)(start + (ok ? t : 0)) * p.x_st + (int64_t)h * p.x_sh + c8;
        if (p.x_dtype == WA_BF16) load8((const bf16_t*)p.x + off, f[r], ok);
        else load8((const float*)p.x + off, f[r], ok);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bf16x4 v4 = {(bf16_t)f[0][e], (bf16_t)f[1][e], (bf16_t)f[2][e], (bf16_t)f[3][e]};
        *(bf16x4*)(xt + (c8 + e) * XLD + tq * 4) = v4;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kc = 0; kc < TC / 16; ++kc) {
      const int tb = t0 + kc * 16 + g * 8;  // tokens of this lane group's fragment
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= mtiles) break;
        const int r = m * 32 + l32;
        bf16x8 af;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = tb + e;
          float v = 0.f;
          if (r < rank && t < seg_len) {
            const int64_t off = (int64_t)r * p.proj_len + t;
            v = p.proj_dtype == WA_BF16 ? (float)((const bf16_t*)p.proj)[off] : ((const float*)p.proj)[off];
          }
          af[e] = (bf16_t)v;
        }
        if (wave_active) {
          const bf16x8 bfr = *(const bf16x8*)(xt + (w * 32 + l32) * XLD + kc * 16 + g * 8);
          acc[m] = wa_mfma32(af, bfr, acc[m]);
        }
      }
    }
  }
  // accumulator: lane holds column d = 32t + l32, rows r = 32m + 8*(i/4) + 4g + i%4
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m >= mtiles) break;
    if (wave_active) {
      const int d = w * 32 + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = m * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        if (r < rank) {
          const int64_t off = (int64_t)b * p.o_sb + (int64_t)(row0 + r) * p.o_st + (int64_t)h * p.o_sh + d;
          wa_store_f(p.out, off, acc[m][i], p.o_dtype);
        }
      }
    }
  }
}

// =============================================================================================
// elu1 state: partial S^T[d, e] = sum_t v[t, d] bf16(phi(k[t, e])) and z[e] over a token range,
// one workgroup per (token chunk, head slot, batch); partials reduced in fixed chunk order.
// =============================================================================================
struct StateParams {
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  int dtype;
  int H, L, D, n_heads, n_chunks, chunk_len;
  const int32_t* heads;
  float* part;     // [n_chunks][B][n_heads][D*D + D]
  float* state; float* zsum;
  int B;
};

template <int D>
__global__ void __launch_bounds__(256) elu1_state_kernel(StateParams p) {
  constexpr int TC = 64;
  constexpr int LD = TC + 8;
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(16))) bf16_t vt[D * LD];
  __shared__ __attribute__((aligned(16))) bf16_t kt[D * LD];
  __shared__ float zred[(TC / 4) * D];
  const int chunk = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int tbeg = chunk * p.chunk_len;
  const int tend = min(p.L, tbeg + p.chunk_len);
  constexpr int UNITS = (TC / 4) * (D / 8);
  const int u = tid;  // one staging unit per thread (UNITS <= 256)
  const int tq = u / (D / 8), c8 = (u % (D / 8)) * 8;
  float zacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) zacc[e] = 0.f;

  // wave w owns d tile w (D <= 128) and every e tile
  const bool wave_active = w < DT;
  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};

  for (int t0 = tbeg; t0 < tend; t0 += TC) {
    __syncthreads();
    if (u < UNITS) {
      float fk[4][8], fv[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + tq * 4 + r;
        const bool ok = t < tend;
        const int tt = ok ? t : tbeg;
        const int64_t ko = (int64_t)b * p.k_sb + (int64_t)tt * p.k_st + (int64_t)h * p.k_sh + c8;
        const int64_t vo = (int64_t)b * p.v_sb + (int64_t)tt * p.v_st + (int64_t)h * p.v_sh + c8;
        if (p.dtype == WA_BF16) {
          load8((const bf16_t*)p.k + ko, fk[r], ok);
          load8((const bf16_t*)p.v + vo, fv[r], ok);
        } else {
          load8((const float*)p.k + ko, fk[r], ok);
          load8((const float*)p.v + vo, fv[r], ok);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float ph = ok ? wa_bf16_round(elu1f(fk[r][e])) : 0.f;
          fk[r][e] = ph;
          zacc[e] += ph;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bf16x4 k4 = {(bf16_t)fk[0][e], (bf16_t)fk[1][e], (bf16_t)fk[2][e], (bf16_t)fk[3][e]};
        bf16x4 v4 = {(bf16_t)fv[0][e], (bf16_t)fv[1][e], (bf16_t)fv[2][e], (bf16_t)fv[3][e]};
        *(bf16x4*)(kt + (c8 + e) * LD + tq * 4) = k4;
        *(bf16x4*)(vt + (c8 + e) * LD + tq * 4) = v4;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kc = 0; kc < TC / 16; ++kc) {
      if (wave_active) {
        const bf16x8 af = *(const bf16x8*)(vt + (w * 32 + l32) * LD + kc * 16 + g * 8);
#pragma unroll
        for (int et = 0; et < DT; ++et) {
          const bf16x8 bfr = *(const bf16x8*)(kt + (et * 32 + l32) * LD + kc * 16 + g * 8);
          acc[et] = wa_mfma32(af, bfr, acc[et]);
        }
      }
    }
  }
  // z partial: reduce the 16 token-quad groups
  if (u < UNITS) {
#pragma unroll
    for (int e = 0; e < 8; ++e) zred[tq * D + c8 + e] = zacc[e];
  }
  __syncthreads();
  float* part = p.part + (((int64_t)chunk * p.B + b) * p.n_heads + hs) * (int64_t)(D * D + D);
  for (int e = tid; e < D; e += 256) {
    float s = 0.f;
    for (int q = 0; q < TC / 4; ++q) s += zred[q * D + e];
    part[D * D + e] = s;
  }
  // S^T partial: accumulator rows = d (8*(i/4) + 4g + i%4 within the tile), columns = e = l32
  if (wave_active) {
#pragma unroll
    for (int et = 0; et < DT; ++et) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = w * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        part[d * D + et * 32 + l32] = acc[et][i];
      }
    }
  }
}

__global__ void __launch_bounds__(256) elu1_reduce_kernel(StateParams p) {
  const int64_t per = (int64_t)p.D * p.D + p.D;
  const int64_t total = (int64_t)p.B * p.n_heads * per;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float s = 0.f;
  for (int c = 0; c < p.n_chunks; ++c) s += p.part[(int64_t)c * total + i];
  const int64_t bh = i / per, r = i % per;
  if (r < (int64_t)p.D * p.D) p.state[bh * p.D * p.D + r] = s;
  else p.zsum[bh * p.D + (r - (int64_t)p.D * p.D)] = s;
}

// =============================================================================================
// elu1 readout: O^T[d, q] = S^T[d, :] phi(Q)^T[:, q] / (phi(q) . z); one workgroup per
// (128-query tile, head slot, batch), wave w owns 32 queries. S^T is split into bf16 hi + lo
// halves (two MFMAs) so the fp32 state keeps ~16 mantissa bits.
// =============================================================================================
struct ReadoutParams {
  const void* q; int64_t q_sb, q_st, q_sh; int q_dtype;
  const float* state; const float* zsum;
  void* o; int64_t o_sb, o_st, o_sh; int o_dtype;
  int H, L, D, n_heads;
  const int32_t* heads;
  int epilogue;
  const bf16_t* gate_w; const float* gate_b;
  int gate_pre_bf16, gate_out_bf16, lin_round_bf16;
};

template <int D>
__global__ void __launch_bounds__(256) elu1_readout_kernel(ReadoutParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  const int tile = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int qi = tile * 128 + w * 32 + l32;
  const bool q_ok = qi < p.L;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)(q_ok ? qi : 0) * p.q_st + (int64_t)h * p.q_sh;
  const float* S = p.state + ((int64_t)b * p.n_heads + hs) * D * D;
  const float* z = p.zsum + ((int64_t)b * p.n_heads + hs) * D;

  bf16x8 qf[DC], phf[DC];
  float den = 0.f;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    float f[8];
    if (p.q_dtype == WA_BF16) load8((const bf16_t*)p.q + qoff + c * 16 + g * 8, f, q_ok);
    else load8((const float*)p.q + qoff + c * 16 + g * 8, f, q_ok);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qf[c][e] = (bf16_t)f[e];
      const float ph = wa_bf16_round(elu1f(f[e]));
      phf[c][e] = (bf16_t)ph;
      den = fmaf(ph, z[c * 16 + g * 8 + e], den);
    }
  }
  den += __shfl_xor(den, 32, 64);

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    oacc[t] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const float* src = S + (int64_t)(t * 32 + l32) * D + c * 16 + g * 8;
      const f32x4 s0 = *(const f32x4*)src, s1 = *(const f32x4*)(src + 4);
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = (bf16_t)s0[e];
        lo[e] = (bf16_t)(s0[e] - (float)hi[e]);
        hi[e + 4] = (bf16_t)s1[e];
        lo[e + 4] = (bf16_t)(s1[e] - (float)hi[e + 4]);
      }
      oacc[t] = wa_mfma32(hi, phf[c], oacc[t]);
      oacc[t] = wa_mfma32(lo, phf[c], oacc[t]);
    }
  }
  f32x16 gacc[DT];
  const bool need_gate = p.epilogue == WA_EPI_GATED;
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
  const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = t * 32 + 8 * rq + 4 * g;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = oacc[t][rq * 4 + i] * inv;
        if (p.lin_round_bf16) a = wa_bf16_round(a);
        if (need_gate) {
          float pre = p.gate_w ? gacc[t][rq * 4 + i] + (p.gate_b ? p.gate_b[d0 + i] : 0.f)
                               : wa_load_f(p.q, qoff + d0 + i, p.q_dtype);
          if (p.gate_pre_bf16) pre = wa_bf16_round(pre);
          float gs = wa_sigmoid(pre);
          if (p.gate_out_bf16) gs = wa_bf16_round(gs);
          a = __fmul_rn(a, gs);
        }
        val[i] = a;
      }
      const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) wa_store_f(p.o, oo + i, val[i], p.o_dtype);
    }
  }
}

int state_chunks(int64_t B, int64_t nh, int64_t L) {
  const int64_t target = 512;
  int64_t per_bh = (target + B * nh - 1) / (B * nh);
  int64_t max_chunks = (L + 63) / 64;
  int64_t c = per_bh < max_chunks ? per_bh : max_chunks;
  return (int)(c < 1 ? 1 : c);
}

}  // namespace

extern "C" int wa_compress_kv(const wa_compress_args* a, void* stream) {
  WA_CHECK_ARG(a && a->x && a->proj && a->out, "wa_compress_kv: null argument");
  WA_CHECK_ARG(a->D == 64 || a->D == 128 || a->D == 32, "wa_compress_kv: head dim %lld not in {32, 64, 128}",
               (long long)a->D);
  WA_CHECK_ARG(a->x_dtype == WA_F32 || a->x_dtype == WA_BF16, "wa_compress_kv: bad dtype");
  WA_CHECK_ARG(a->proj_dtype == WA_F32 || a->proj_dtype == WA_BF16, "wa_compress_kv: bad proj dtype");
  WA_CHECK_ARG(a->segment_len > 0 && a->block_size > 0 && a->L > 0, "wa_compress_kv: bad sizes");
  WA_CHECK_ARG(a->proj_rank > 0 && a->proj_rank <= 128, "wa_compress_kv: projection rank must be in [1, 128]");
  const int64_t nseg = (a->L + a->segment_len - 1) / a->segment_len;
  const int64_t first_seg = a->segment_len < a->L ? a->segment_len : a->L;
  WA_CHECK_ARG(first_seg <= a->proj_len, "wa_compress_kv: segment length %lld exceeds projection length %lld",
               (long long)first_seg, (long long)a->proj_len);
  if (a->B == 0) return WA_OK;
  CompressParams cp{a->x, a->x_sb, a->x_st, a->x_sh, a->x_dtype, a->proj, a->proj_dtype, (int)a->proj_rank,
                    (int)a->proj_len, (int)a->L, (int)a->H, (int)a->D, (int)a->segment_len, (int)a->block_size,
                    a->out, a->o_sb, a->o_st, a->o_sh, a->o_dtype};
  dim3 grid((unsigned)nseg, (unsigned)a->H, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(compress_kernel<128>, grid, dim3(256), 0, s, cp);
  else if (a->D == 64) hipLaunchKernelGGL(compress_kernel<64>, grid, dim3(256), 0, s, cp);
  else hipLaunchKernelGGL(compress_kernel<32>, grid, dim3(256), 0, s, cp);
  return wa_launch_status("compress_kv");
}

extern "C" int64_t wa_elu1_state_workspace_bytes(int64_t B, int64_t n_heads, int64_t L, int64_t D) {
  const int64_t chunks = state_chunks(B, n_heads, L);
  return ((chunks * B * n_heads * (D * D + D)) * 4 + 255) / 256 * 256;
}

extern "C" int wa_elu1_state(const wa_elu1_state_args* a, void* stream) {
  WA_CHECK_ARG(a && a->k && a->v && a->state && a->zsum && a->workspace, "wa_elu1_state: null argument");
  WA_CHECK_ARG(a->D == 64 || a->D == 128 || a->D == 32, "wa_elu1_state: head dim %lld not in {32, 64, 128}",
               (long long)a->D);
  WA_CHECK_ARG(a->dtype == WA_F32 || a->dtype == WA_BF16, "wa_elu1_state: bad dtype");
  WA_CHECK_ARG(a->L > 0 && a->H > 0 && a->B >= 0, "wa_elu1_state: bad sizes");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || nh == 0) return WA_OK;
  StateParams sp{};
  sp.k = a->k; sp.k_sb = a->k_sb; sp.k_st = a->k_st; sp.k_sh = a->k_sh;
  sp.v = a->v; sp.v_sb = a->v_sb; sp.v_st = a->v_st; sp.v_sh = a->v_sh;
  sp.dtype = a->dtype; sp.H = (int)a->H; sp.L = (int)a->L; sp.D = (int)a->D; sp.n_heads = (int)nh;
  sp.n_chunks = state_chunks(a->B, nh, a->L);
  sp.chunk_len = (int)(((a->L + sp.n_chunks - 1) / sp.n_chunks + 63) / 64 * 64);
  sp.n_chunks = (int)((a->L + sp.chunk_len - 1) / sp.chunk_len);
  sp.heads = a->heads; sp.part = (float*)a->workspace; sp.state = a->state; sp.zsum = a->zsum; sp.B = (int)a->B;
  dim3 grid((unsigned)sp.n_chunks, (unsigned)nh, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(elu1_state_kernel<128>, grid, dim3(256), 0, s, sp);
  else if (a->D == 64) hipLaunchKernelGGL(elu1_state_kernel<64>, grid, dim3(256), 0, s, sp);
  else hipLaunchKernelGGL(elu1_state_kernel<32>, grid, dim3(256), 0, s, sp);
  int rc = wa_launch_status("elu1_state");
  if (rc != WA_OK) return rc;
  const int64_t total = a->B * nh * (a->D * a->D + a->D);
  hipLaunchKernelGGL(elu1_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, sp);
  return wa_launch_status("elu1_reduce");
}

extern "C" int wa_elu1_readout(const wa_elu1_readout_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->state && a->zsum && a->o, "wa_elu1_readout: null argument");
  WA_CHECK_ARG(a->D == 64 || a->D == 128 || a->D == 32, "wa_elu1_readout: head dim %lld not in {32, 64, 128}",
               (long long)a->D);
  WA_CHECK_ARG(a->q_dtype == WA_F32 || a->q_dtype == WA_BF16, "wa_elu1_readout: bad q dtype");
  WA_CHECK_ARG(a->o_dtype == WA_F32 || a->o_dtype == WA_BF16, "wa_elu1_readout: bad o dtype");
  WA_CHECK_ARG(a->epilogue == WA_EPI_PLAIN || a->epilogue == WA_EPI_GATED, "wa_elu1_readout: epilogue must be PLAIN or GATED");
  WA_CHECK_ARG(wa_aligned16(a->state), "wa_elu1_readout: state must be 16-byte aligned");
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "wa_elu1_readout: gate_w must be 16-byte aligned");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || nh == 0 || a->L == 0) return WA_OK;
  ReadoutParams rp{a->q, a->q_sb, a->q_st, a->q_sh, a->q_dtype, a->state, a->zsum, a->o, a->o_sb, a->o_st,
                   a->o_sh, a->o_dtype, (int)a->H, (int)a->L, (int)a->D, (int)nh, a->heads, a->epilogue,
                   (const bf16_t*)a->gate_w, a->gate_b, a->gate_pre_bf16, a->gate_out_bf16, a->lin_round_bf16};
  dim3 grid((unsigned)((a->L + 127) / 128), (unsigned)nh, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) hipLaunchKernelGGL(elu1_readout_kernel<128>, grid, dim3(256), 0, s, rp);
  else if (a->D == 64) hipLaunchKernelGGL(elu1_readout_kernel<64>, grid, dim3(256), 0, s, rp);
  else hipLaunchKernelGGL(elu1_readout_kernel<32>, grid, dim3(256), 0, s, rp);
  return wa_launch_status("elu1_readout");
}
