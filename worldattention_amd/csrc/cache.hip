// KV-cache write side of a causal attention step: appending a chunk's keys and values, the fused
// QKV epilogue (RMSNorm + 3-D RoPE + cache write), the sliding-window roll, and the key block sums
// the routing reads instead of pooling the keys.
//
// Reference semantics: wan/modules/causal_model.py:34-62 (causal_rope_apply), :166-169 with
// wan/modules/model.py:70-86 (WanRMSNorm), :286-437 (cache roll / insert in the step) and
// :1016-1119 (the same updates at commit).
#include <algorithm>

#include "common.h"
#include "torch_order.h"

namespace {

// ---------------------------------------------------------------------------------------------
// Copies of [B, n, H, D] BLHD tensors, 16 bytes per thread; blockIdx.y picks one of up to two
// (source, destination) pairs of one launch.
// ---------------------------------------------------------------------------------------------
struct CopyPair {
  const void* src; int64_t s_sb, s_st, s_sh;
  void* dst; int64_t d_sb, d_st, d_sh;
};

template <typename T, int VEC>
__global__ void __launch_bounds__(256) kv_copy_kernel(CopyPair c0, CopyPair c1, int B, int n, int H, int D) {
  const CopyPair& c = blockIdx.y ? c1 : c0;
  const int64_t cpr = D / VEC;  // chunks per head row
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)B * n * H * cpr;
  if (i >= total) return;
  const int ch = (int)(i % cpr);
  const int64_t r = i / cpr;
  const int h = (int)(r % H), t = (int)((r / H) % n), b = (int)(r / ((int64_t)H * n));
  const T* sp = (const T*)c.src + b * c.s_sb + t * c.s_st + h * c.s_sh + ch * VEC;
  T* dp = (T*)c.dst + b * c.d_sb + t * c.d_st + h * c.d_sh + ch * VEC;
  if constexpr (VEC * sizeof(T) == 16) {
    *(u32x4*)dp = *(const u32x4*)sp;
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) dp[e] = sp[e];
  }
}

bool pair_vec16(const CopyPair& c, int vec, int64_t D) {
  return wa_aligned16(c.src) && wa_aligned16(c.dst) && D % vec == 0 && c.s_sb % vec == 0 && c.s_st % vec == 0 &&
         c.s_sh % vec == 0 && c.d_sb % vec == 0 && c.d_st % vec == 0 && c.d_sh % vec == 0;
}

// One launch copying n tokens of each pair (the second pair may have src == NULL: one pair only).
int kv_copy(const CopyPair& c0, const CopyPair& c1, int dtype, int64_t B, int64_t n, int64_t H, int64_t D,
            hipStream_t s) {
  const int es = dtype == WA_BF16 ? 2 : 4, vec = 16 / es;
  const bool two = c1.src != nullptr;
  const bool v16 = pair_vec16(c0, vec, D) && (!two || pair_vec16(c1, vec, D));
  const int64_t total = B * n * H * (v16 ? D / vec : D);
  if (total == 0) return WA_OK;
  const dim3 grid((unsigned)((total + 255) / 256), two ? 2u : 1u);
  if (dtype == WA_BF16) {
    if (v16) hipLaunchKernelGGL((kv_copy_kernel<bf16_t, 8>), grid, dim3(256), 0, s, c0, c1, (int)B, (int)n, (int)H, (int)D);
    else hipLaunchKernelGGL((kv_copy_kernel<bf16_t, 1>), grid, dim3(256), 0, s, c0, c1, (int)B, (int)n, (int)H, (int)D);
  } else {
    if (v16) hipLaunchKernelGGL((kv_copy_kernel<float, 4>), grid, dim3(256), 0, s, c0, c1, (int)B, (int)n, (int)H, (int)D);
    else hipLaunchKernelGGL((kv_copy_kernel<float, 1>), grid, dim3(256), 0, s, c0, c1, (int)B, (int)n, (int)H, (int)D);
  }
  return wa_launch_status("kv_copy");
}

// ---------------------------------------------------------------------------------------------
// QKV epilogue. Workgroups [0, q_jobs) take TT query tokens each (all heads); the rest take TT
// written key/value tokens each. A token row is its H*D channels: the RMSNorm mean runs over the
// row in torch's CPU fp32 order (8 lanes of stride 8 summed by 8 threads, then the tail and the
// lanes in order by one), staged in LDS; the RoPE pairs (2c, 2c+1) of each head rotate by the
// table entry of the band c falls in (temporal: frame start_frame + f, height: row h, width:
// column w of the token's grid position).
// ---------------------------------------------------------------------------------------------
struct EpiParams {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  void* qo; int64_t qo_sb, qo_st, qo_sh;
  void* ck; int64_t ck_sb, ck_st, ck_sh;
  void* cv; int64_t cv_sb, cv_st, cv_sh;
  int B, n, H, D, HD;
  int write_start, src_offset, write_len;
  const double* freqs;
  int gf, gh, gw, start_frame, seq_len, ct, ch;
  const void* qw; const void* kw; int w_bf16; float eps;
  int TT, q_tiles, kv_tiles;
};

__device__ __forceinline__ void rope_pair(double a, double b, const double* f, double& re, double& im) {
#pragma clang fp contract(off)
  // (a + ib)(c + id) with each product rounded, then one add (torch's complex128 product)
  const double c = f[0], d = f[1];
  const double ac = a * c, bd = b * d, ad = a * d, bc = b * c;
  re = ac - bd;
  im = ad + bc;
}

template <typename T>
__device__ __forceinline__ float epi_to_float(T x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T epi_from_double(double x) {
  // the reference's double -> output dtype: to fp32 (nearest), then to the dtype (nearest even)
  return (T)(float)x;
}

// Row r of the TT rows: RMSNorm factor 1 / sqrt(mean(x^2) + eps) in torch's fp32 order.
template <typename T>
__device__ void epi_norm_factors(const EpiParams& p, const T* stage, int rows, float* part, float* rs) {
  const int tid = threadIdx.x;
  const int HD = p.HD, nv = HD / 8;
  if (tid < rows * 8) {
    const int r = tid >> 3, l = tid & 7;
    const T* row = stage + (int64_t)r * HD;
    auto sq = [&](int i) {
      const float x = epi_to_float(row[i]);
      return wa_mul_rn(x, x);
    };
    part[r * 8 + l] = nv > 0 ? tc_row_sum(sq, l, 8, nv) : 0.f;
  }
  __syncthreads();
  if (tid < rows) {
    const T* row = stage + (int64_t)tid * HD;
    auto sq = [&](int i) {
      const float x = epi_to_float(row[i]);
      return wa_mul_rn(x, x);
    };
    float fin;
    if (HD < 8) {
      fin = tc_row_sum(sq, 0, 1, HD);
    } else {
      fin = 0.f;
      for (int i = nv * 8; i < HD; ++i) fin = wa_add_rn(fin, sq(i));
      for (int l = 0; l < 8; ++l) fin = wa_add_rn(fin, part[tid * 8 + l]);
    }
    const float mean = wa_div_rn(fin, (float)HD);
    // sqrtf, not __fsqrt_rn: on gfx950 the latter is the bare v_sqrt_f32 (about 1 ulp), sqrtf
    // adds the correction that makes it correctly rounded, as torch's CPU sqrt is
    rs[tid] = wa_div_rn(1.f, sqrtf(wa_add_rn(mean, p.eps)));
  }
  __syncthreads();
}

// Normalize (optional) and rotate TT token rows of one tensor: source tokens s0 .. s0 + rows - 1
// (RoPE position s = source token), written to destination tokens d0 .. of dst.
template <typename T>
__device__ void epi_rows(const EpiParams& p, const T* src, int64_t s_sb, int64_t s_st, int64_t s_sh, T* dst,
                         int64_t d_sb, int64_t d_st, int64_t d_sh, int b, int s0, int d0, int rows,
                         const void* w, bool rope, T* stage, float* part, float* rs) {
  constexpr int VEC = 16 / sizeof(T);
  const int tid = threadIdx.x, D = p.D, HD = p.HD, cpr = HD / VEC;
  const int half = D / 2;
  const T* sbase = src + (int64_t)b * s_sb;
  T* dbase = dst + (int64_t)b * d_sb;
  auto src_at = [&](int r, int e) { const int h = e / D, d = e - h * D; return sbase + (int64_t)(s0 + r) * s_st + (int64_t)h * s_sh + d; };
  if (w) {
    for (int u = tid; u < rows * cpr; u += 256) {
      const int r = u / cpr, e = (u - r * cpr) * VEC;
      *(u32x4*)(stage + (int64_t)r * HD + e) = *(const u32x4*)src_at(r, e);
    }
    __syncthreads();
    epi_norm_factors<T>(p, stage, rows, part, rs);
  }
  for (int u = tid; u < rows * cpr; u += 256) {
    const int r = u / cpr, e = (u - r * cpr) * VEC;
    const int h = e / D, d = e - h * D;
    T x[VEC];
    if (w) *(u32x4*)x = *(const u32x4*)(stage + (int64_t)r * HD + e);
    else *(u32x4*)x = *(const u32x4*)src_at(r, e);
    float y[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      y[i] = epi_to_float(x[i]);
      if (w) {
        // x * rsqrt(...) in fp32, rounded to the input dtype, times the weight in the wider dtype
        const float nx = (float)(T)wa_mul_rn(y[i], rs[r]);
        if (p.w_bf16) {
          const float wv = (float)((const bf16_t*)w)[e + i];
          y[i] = sizeof(T) == 2 ? (float)(T)wa_mul_rn(nx, wv) : wa_mul_rn(nx, wv);
        } else {
          y[i] = wa_mul_rn(nx, ((const float*)w)[e + i]);
        }
      }
    }
    const int s = s0 + r;
    T out[VEC];
    if (rope && s < p.seq_len) {
      const int fi = s / (p.gh * p.gw), rem = s - fi * p.gh * p.gw, hi = rem / p.gw, wi = rem - hi * p.gw;
#pragma unroll
      for (int i = 0; i < VEC; i += 2) {
        const int c = (d + i) >> 1;
        const int row = c < p.ct ? p.start_frame + fi : (c < p.ct + p.ch ? hi : wi);
        double re, im;
        rope_pair((double)y[i], (double)y[i + 1], p.freqs + ((int64_t)row * half + c) * 2, re, im);
        out[i] = epi_from_double<T>(re);
        out[i + 1] = epi_from_double<T>(im);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) out[i] = (T)y[i];
    }
    *(u32x4*)(dbase + (int64_t)(d0 + r) * d_st + (int64_t)h * d_sh + d) = *(const u32x4*)out;
  }
  if (w) __syncthreads();  // the stage is reused by the next tensor
}

template <typename T>
__global__ void __launch_bounds__(256) qkv_epilogue_kernel(EpiParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char epi_lds[];
  T* stage = (T*)epi_lds;
  float* part = (float*)(epi_lds + (int64_t)p.TT * p.HD * sizeof(T));
  float* rs = part + p.TT * 8;
  int job = blockIdx.x;
  if (job < p.B * p.q_tiles) {
    const int b = job / p.q_tiles, s0 = (job % p.q_tiles) * p.TT;
    const int rows = min(p.TT, p.n - s0);
    epi_rows<T>(p, (const T*)p.q, p.q_sb, p.q_st, p.q_sh, (T*)p.qo, p.qo_sb, p.qo_st, p.qo_sh, b, s0, s0, rows, p.qw,
                true, stage, part, rs);
    return;
  }
  job -= p.B * p.q_tiles;
  const int b = job / p.kv_tiles, t0 = (job % p.kv_tiles) * p.TT;
  const int rows = min(p.TT, p.write_len - t0);
  epi_rows<T>(p, (const T*)p.k, p.k_sb, p.k_st, p.k_sh, (T*)p.ck, p.ck_sb, p.ck_st, p.ck_sh, b, p.src_offset + t0,
              p.write_start + t0, rows, p.kw, true, stage, part, rs);
  epi_rows<T>(p, (const T*)p.v, p.v_sb, p.v_st, p.v_sh, (T*)p.cv, p.cv_sb, p.cv_st, p.cv_sh, b, p.src_offset + t0,
              p.write_start + t0, rows, nullptr, false, stage, part, rs);
}

bool blhd_vec_ok(const void* ptr, int64_t sb, int64_t st, int64_t sh, int vec) {
  return wa_aligned16(ptr) && sb % vec == 0 && st % vec == 0 && sh % vec == 0;
}

}  // namespace

extern "C" int wa_kv_append(const wa_kv_append_args* a, void* stream) {
  WA_CHECK_ARG(a && a->cache_k && a->cache_v && a->new_k && a->new_v, "wa_kv_append: null argument");
  WA_CHECK_ARG(a->dtype == WA_BF16 || a->dtype == WA_F32, "wa_kv_append: dtype must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->D > 0 && a->cap > 0 && a->n >= 0 && a->start >= 0 &&
                   a->start + a->n <= a->cap,
               "wa_kv_append: tokens [%lld, %lld) do not fit a cache of %lld", (long long)a->start,
               (long long)(a->start + a->n), (long long)a->cap);
  WA_CHECK_ARG(a->B < (1 << 20) && a->cap < ((int64_t)1 << 30) && a->H < (1 << 16) && a->D <= 1024,
               "wa_kv_append: sizes too large");
  if (a->B == 0 || a->n == 0) return WA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t es = a->dtype == WA_BF16 ? 2 : 4;
  // token `start` of each cache
  const CopyPair ck{a->new_k, a->nk_sb, a->nk_st, a->nk_sh, (char*)a->cache_k + a->start * a->ck_st * es,
                    a->ck_sb, a->ck_st, a->ck_sh};
  const CopyPair cv{a->new_v, a->nv_sb, a->nv_st, a->nv_sh, (char*)a->cache_v + a->start * a->cv_st * es,
                    a->cv_sb, a->cv_st, a->cv_sh};
  int rc = kv_copy(ck, cv, a->dtype, a->B, a->n, a->H, a->D, s);
  if (rc != WA_OK) return rc;
  // sums of the key blocks that hold a new token, over the cache tokens [0, start + n)
  if (!a->k_sums) return WA_OK;
  WA_CHECK_ARG(a->block_size > 0, "wa_kv_append: k_sums needs a block size");
  const int64_t first = a->start / a->block_size, L = a->start + a->n;
  wa_pool_args pa{};
  pa.x = a->cache_k; pa.x_sb = a->ck_sb; pa.x_st = a->ck_st; pa.x_sh = a->ck_sh; pa.x_dtype = a->dtype;
  pa.B = a->B; pa.L = L; pa.H = a->H; pa.D = a->D; pa.block_size = a->block_size;
  pa.first_block = first;
  pa.num_blocks = (L + a->block_size - 1) / a->block_size - first;
  pa.heads = a->heads; pa.n_heads = a->n_heads;
  pa.out = a->k_sums; pa.out_blocks = (a->cap + a->block_size - 1) / a->block_size;
  pa.emulate_rounding = 1; pa.store_sums = 1;
  return wa_block_mean_pool(&pa, s);
}

extern "C" int wa_qkv_epilogue(const wa_qkv_epilogue_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->k && a->v && a->q_out && a->cache_k && a->cache_v && a->freqs,
               "wa_qkv_epilogue: null argument");
  WA_CHECK_ARG(a->dtype == WA_BF16 || a->dtype == WA_F32, "wa_qkv_epilogue: dtype must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 0 && a->n >= 0 && a->H > 0 && a->D > 0 && a->D % 8 == 0 && a->D <= 1024,
               "wa_qkv_epilogue: head dim must be a multiple of 8 up to 1024");
  WA_CHECK_ARG(a->B < (1 << 20) && a->n < (1 << 30) && a->H < (1 << 16) && a->cap < ((int64_t)1 << 30),
               "wa_qkv_epilogue: sizes too large");
  WA_CHECK_ARG(a->write_len >= 0 && a->src_offset >= 0 && a->src_offset + a->write_len <= a->n &&
                   a->write_start >= 0 && a->write_start + a->write_len <= a->cap,
               "wa_qkv_epilogue: write of %lld tokens from %lld to cache token %lld does not fit (n %lld, cap %lld)",
               (long long)a->write_len, (long long)a->src_offset, (long long)a->write_start, (long long)a->n,
               (long long)a->cap);
  // the grid of sample b (every sample's when sample_grids is NULL)
  auto grid_of = [&](int64_t b, int64_t* g) {
    const int64_t* src = a->sample_grids ? a->sample_grids + 3 * b : nullptr;
    g[0] = src ? src[0] : a->grid_f;
    g[1] = src ? src[1] : a->grid_h;
    g[2] = src ? src[2] : a->grid_w;
  };
  for (int64_t b = 0; b < (a->sample_grids ? a->B : 1); ++b) {
    int64_t g[3];
    grid_of(b, g);
    WA_CHECK_ARG(g[0] >= 0 && g[1] > 0 && g[2] > 0 && a->start_frame >= 0, "wa_qkv_epilogue: bad grid");
    WA_CHECK_ARG(g[0] * g[1] * g[2] <= a->n, "wa_qkv_epilogue: grid of %lld tokens exceeds the %lld tokens given",
                 (long long)(g[0] * g[1] * g[2]), (long long)a->n);
    WA_CHECK_ARG(a->start_frame + g[0] <= a->f_rows && g[1] <= a->f_rows && g[2] <= a->f_rows,
                 "wa_qkv_epilogue: grid positions beyond the %lld rows of the RoPE table", (long long)a->f_rows);
  }
  WA_CHECK_ARG(((uintptr_t)a->freqs & 15u) == 0, "wa_qkv_epilogue: freqs must be 16-byte aligned");
  const bool norm = a->q_norm_w || a->k_norm_w;
  WA_CHECK_ARG(!norm || (a->q_norm_w && a->k_norm_w && (a->w_dtype == WA_BF16 || a->w_dtype == WA_F32)),
               "wa_qkv_epilogue: give both norm weights (bf16 or fp32) or neither");
  const int vec = a->dtype == WA_BF16 ? 8 : 4;
  WA_CHECK_ARG(blhd_vec_ok(a->q, a->q_sb, a->q_st, a->q_sh, vec) && blhd_vec_ok(a->k, a->k_sb, a->k_st, a->k_sh, vec) &&
                   blhd_vec_ok(a->v, a->v_sb, a->v_st, a->v_sh, vec) &&
                   blhd_vec_ok(a->q_out, a->qo_sb, a->qo_st, a->qo_sh, vec) &&
                   blhd_vec_ok(a->cache_k, a->ck_sb, a->ck_st, a->ck_sh, vec) &&
                   blhd_vec_ok(a->cache_v, a->cv_sb, a->cv_st, a->cv_sh, vec),
               "wa_qkv_epilogue: tensors must be 16-byte aligned with 16-byte aligned rows");
  if (a->B == 0 || a->n == 0) return WA_OK;
  const int64_t es = a->dtype == WA_BF16 ? 2 : 4, HD = a->H * a->D;
  const int TT = (int)std::max<int64_t>(1, std::min<int64_t>(16, 65536 / (HD * es)));
  WA_CHECK_ARG(HD * es * TT <= 65536 || TT == 1, "wa_qkv_epilogue: token row too long");
  WA_CHECK_ARG(HD * es <= 96 * 1024, "wa_qkv_epilogue: a token row of %lld bytes exceeds the LDS stage",
               (long long)(HD * es));
  EpiParams p{};
  p.q = a->q; p.q_sb = a->q_sb; p.q_st = a->q_st; p.q_sh = a->q_sh;
  p.k = a->k; p.k_sb = a->k_sb; p.k_st = a->k_st; p.k_sh = a->k_sh;
  p.v = a->v; p.v_sb = a->v_sb; p.v_st = a->v_st; p.v_sh = a->v_sh;
  p.qo = a->q_out; p.qo_sb = a->qo_sb; p.qo_st = a->qo_st; p.qo_sh = a->qo_sh;
  p.ck = a->cache_k; p.ck_sb = a->ck_sb; p.ck_st = a->ck_st; p.ck_sh = a->ck_sh;
  p.cv = a->cache_v; p.cv_sb = a->cv_sb; p.cv_st = a->cv_st; p.cv_sh = a->cv_sh;
  p.B = (int)a->B; p.n = (int)a->n; p.H = (int)a->H; p.D = (int)a->D; p.HD = (int)HD;
  p.write_start = (int)a->write_start; p.src_offset = (int)a->src_offset; p.write_len = (int)a->write_len;
  p.freqs = a->freqs;
  p.start_frame = (int)a->start_frame;
  const int half = (int)(a->D / 2);
  p.ct = half - 2 * (half / 3); p.ch = half / 3;
  p.qw = a->q_norm_w; p.kw = a->k_norm_w; p.w_bf16 = a->w_dtype == WA_BF16; p.eps = a->eps;
  p.TT = TT;
  p.q_tiles = (int)((a->n + TT - 1) / TT);
  p.kv_tiles = (int)((a->write_len + TT - 1) / TT);
  WA_CHECK_ARG(a->B * (p.q_tiles + p.kv_tiles) < ((int64_t)1 << 31), "wa_qkv_epilogue: too many tokens for one launch");
  const size_t lds = norm ? (size_t)TT * HD * es + (size_t)TT * 9 * sizeof(float) : 16;
  hipStream_t s = (hipStream_t)stream;
  // one launch per run of consecutive samples that share a grid (the whole batch without
  // sample_grids): pointers moved to the run's first sample, B = its length
  const int64_t el = es;
  int rc = WA_OK;
  for (int64_t b0 = 0; b0 < a->B && rc == WA_OK;) {
    int64_t g[3], gn[3];
    grid_of(b0, g);
    int64_t b1 = b0 + 1;
    if (a->sample_grids) {
      for (; b1 < a->B; ++b1) {
        grid_of(b1, gn);
        if (gn[0] != g[0] || gn[1] != g[1] || gn[2] != g[2]) break;
      }
    } else {
      b1 = a->B;
    }
    EpiParams pr = p;
    pr.q = (const char*)a->q + b0 * a->q_sb * el;
    pr.k = (const char*)a->k + b0 * a->k_sb * el;
    pr.v = (const char*)a->v + b0 * a->v_sb * el;
    pr.qo = (char*)a->q_out + b0 * a->qo_sb * el;
    pr.ck = (char*)a->cache_k + b0 * a->ck_sb * el;
    pr.cv = (char*)a->cache_v + b0 * a->cv_sb * el;
    pr.B = (int)(b1 - b0);
    pr.gf = (int)g[0]; pr.gh = (int)g[1]; pr.gw = (int)g[2];
    pr.seq_len = (int)(g[0] * g[1] * g[2]);
    const int64_t jobs = (b1 - b0) * (p.q_tiles + p.kv_tiles);
    if (a->dtype == WA_BF16)
      hipLaunchKernelGGL(qkv_epilogue_kernel<bf16_t>, dim3((unsigned)jobs), dim3(256), lds, s, pr);
    else
      hipLaunchKernelGGL(qkv_epilogue_kernel<float>, dim3((unsigned)jobs), dim3(256), lds, s, pr);
    rc = wa_launch_status("qkv_epilogue");
    b0 = b1;
  }
  if (rc != WA_OK || !a->k_sums || a->write_len == 0) return rc;
  WA_CHECK_ARG(a->block_size > 0, "wa_qkv_epilogue: k_sums needs a block size");
  const int64_t L = a->write_start + a->write_len, first = a->write_start / a->block_size;
  wa_pool_args pa{};
  pa.x = a->cache_k; pa.x_sb = a->ck_sb; pa.x_st = a->ck_st; pa.x_sh = a->ck_sh; pa.x_dtype = a->dtype;
  pa.B = a->B; pa.L = L; pa.H = a->H; pa.D = a->D; pa.block_size = a->block_size;
  pa.first_block = first;
  pa.num_blocks = (L + a->block_size - 1) / a->block_size - first;
  pa.out = a->k_sums; pa.out_blocks = (a->cap + a->block_size - 1) / a->block_size;
  pa.emulate_rounding = 1; pa.store_sums = 1;
  return wa_block_mean_pool(&pa, s);
}

extern "C" int wa_kv_roll(const wa_kv_roll_args* a, void* stream) {
  WA_CHECK_ARG(a && a->cache_k && a->cache_v, "wa_kv_roll: null argument");
  WA_CHECK_ARG(a->dtype == WA_BF16 || a->dtype == WA_F32, "wa_kv_roll: dtype must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->D > 0 && a->D <= 1024 && a->cap > 0, "wa_kv_roll: bad sizes");
  WA_CHECK_ARG(a->sink >= 0 && a->evicted >= 0 && a->rolled >= 0 && a->sink + a->evicted + a->rolled <= a->cap,
               "wa_kv_roll: tokens [%lld, %lld) beyond a cache of %lld", (long long)(a->sink + a->evicted),
               (long long)(a->sink + a->evicted + a->rolled), (long long)a->cap);
  const bool coarse = a->k_coarse || a->v_coarse;
  if (coarse)
    WA_CHECK_ARG(a->k_coarse && a->v_coarse && a->c_rows >= 0 && a->c_dst >= 0 && a->c_src >= a->c_dst &&
                     a->c_src + a->c_rows <= a->coarse_cap,
                 "wa_kv_roll: bad coarse rows");
  if (a->B == 0) return WA_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t es = a->dtype == WA_BF16 ? 2 : 4;
  // Tokens move left by `evicted`. Each launch copies at most `evicted` tokens, so its destination
  // is what earlier launches already read: no launch overwrites tokens another still has to read.
  auto roll = [&](void* k, int64_t ksb, int64_t kst, int64_t ksh, void* v, int64_t vsb, int64_t vst, int64_t vsh,
                  int64_t dst0, int64_t shift, int64_t count) -> int {
    if (shift == 0 || count == 0) return WA_OK;
    for (int64_t off = 0; off < count; off += shift) {
      const int64_t m = std::min(shift, count - off);
      const CopyPair ck{(char*)k + (dst0 + shift + off) * kst * es, ksb, kst, ksh,
                        (char*)k + (dst0 + off) * kst * es, ksb, kst, ksh};
      const CopyPair cv{(char*)v + (dst0 + shift + off) * vst * es, vsb, vst, vsh,
                        (char*)v + (dst0 + off) * vst * es, vsb, vst, vsh};
      const int rc = kv_copy(ck, cv, a->dtype, a->B, m, a->H, a->D, s);
      if (rc != WA_OK) return rc;
    }
    return WA_OK;
  };
  int rc = roll(a->cache_k, a->ck_sb, a->ck_st, a->ck_sh, a->cache_v, a->cv_sb, a->cv_st, a->cv_sh, a->sink,
                a->evicted, a->rolled);
  if (rc != WA_OK) return rc;
  if (coarse) {
    rc = roll(a->k_coarse, a->kc_sb, a->kc_st, a->kc_sh, a->v_coarse, a->vc_sb, a->vc_st, a->vc_sh, a->c_dst,
              a->c_src - a->c_dst, a->c_rows);
    if (rc != WA_OK) return rc;
  }
  if (!a->k_sums || a->rolled == 0 || a->evicted == 0) return WA_OK;
  WA_CHECK_ARG(a->block_size > 0, "wa_kv_roll: k_sums needs a block size");
  const int64_t L = a->sink + a->rolled, first = a->sink / a->block_size;
  wa_pool_args pa{};
  pa.x = a->cache_k; pa.x_sb = a->ck_sb; pa.x_st = a->ck_st; pa.x_sh = a->ck_sh; pa.x_dtype = a->dtype;
  pa.B = a->B; pa.L = L; pa.H = a->H; pa.D = a->D; pa.block_size = a->block_size;
  pa.first_block = first;
  pa.num_blocks = (L + a->block_size - 1) / a->block_size - first;
  pa.heads = a->heads; pa.n_heads = a->n_heads;
  pa.out = a->k_sums; pa.out_blocks = (a->cap + a->block_size - 1) / a->block_size;
  pa.emulate_rounding = 1; pa.store_sums = 1;
  return wa_block_mean_pool(&pa, s);
}
