// Low-rank linear branch of the reference (wan/modules/hsa/attention.py:64-118) for gfx950:
//  * compress_kv — low-rank sequence projection per segment (attention.py:64-110); the softmax
//    over the compressed keys then runs in the block-sparse kernel as dense attention.
// The contraction runs on v_mfma_f32_32x32x16_bf16 with fp32 accumulation; the token-axis
// operand is staged through LDS transposed ([channel][token]).
// The north-star elu(x)+1 linear branch lives in elu1.hip.
#include "common.h"

namespace {

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
