// HKV tier kernels for gfx950 (pipeline/hkv of the reference):
//  * page summary  — de-roped per-page mean keys, query / prompt means (one HBM pass + a tiny
//                    fixed-order reduction);
//  * score + top-k — page affinities and a bitonic top-k (lowest page index wins ties) in one
//                    workgroup;
//  * rerope        — temporal-band rotation of installed pages (only the band is touched in place);
//  * page copies   — pinned host <-> device 2-D copies enqueued on the caller's side stream.
#include <math.h>

#include <algorithm>

#include <vector>

#include "common.h"

namespace {

// ---------------------------------------------------------------------------------------------
// Vector access of VEC consecutive channels (VEC = 8: 16-byte aligned runs; VEC = 2 or 1: any).
// ---------------------------------------------------------------------------------------------
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float (&f)[VEC]) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    const bf16x8 v = *(const bf16x8*)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
  } else if constexpr (VEC == 8) {
    const f32x4 a = *(const f32x4*)p, b = *((const f32x4*)p + 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) { f[e] = a[e]; f[4 + e] = b[e]; }
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) f[e] = (float)p[e];
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float (&f)[VEC]) {
  if constexpr (VEC == 8 && sizeof(T) == 2) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16_t)f[e];
    *(bf16x8*)p = v;
  } else if constexpr (VEC == 8) {
    *(f32x4*)p = f32x4{f[0], f[1], f[2], f[3]};
    *((f32x4*)p + 1) = f32x4{f[4], f[5], f[6], f[7]};
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) p[e] = (T)f[e];
  }
}

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (sizeof(T) == 2) return wa_bf16_round(x);
  else return x;
}

// Multiplies the complex pairs of f (channels d0 .. d0 + VEC of a head) that lie in the temporal
// band (pair < nt) by the factor row, in fp32, and rounds each result to T. The products and sums
// round separately (no fused multiply-add the compiler may or may not form), so every kernel that
// rotates keys gives the same bits.
template <typename T, int VEC>
__device__ __forceinline__ void rotate_band(float (&f)[VEC], int d0, const float2* frow, int nt) {
  static_assert(VEC % 2 == 0, "rotation works on whole complex pairs");
#pragma unroll
  for (int e = 0; e < VEC; e += 2) {
    const int pr = (d0 + e) >> 1;
    if (pr < nt) {
      const float2 w = frow[pr];
      const float re = wa_sub_rn(wa_mul_rn(f[e], w.x), wa_mul_rn(f[e + 1], w.y));
      const float im = wa_add_rn(wa_mul_rn(f[e], w.y), wa_mul_rn(f[e + 1], w.x));
      f[e] = round_to<T>(re);
      f[e + 1] = round_to<T>(im);
    }
  }
}

// =============================================================================================
// Page summary: partial column sums per (segment, batch, token split), then a fixed-order
// reduction per segment. One thread owns VEC consecutive channels of one head.
// =============================================================================================
// 256 tokens per split: one round of workgroups at the cfg 3 shape (120 pages x 7 splits); 64 made
// 3,000 workgroups of which the last ~440 ran a second, nearly empty round (125 -> 116 us).
constexpr int SUM_TOKENS_PER_SPLIT = 256;
constexpr int SUM_MAX_SPLITS = 64;

int64_t summary_splits(int64_t max_seg_tokens) {
  const int64_t s = (std::max<int64_t>(max_seg_tokens, 1) + SUM_TOKENS_PER_SPLIT - 1) / SUM_TOKENS_PER_SPLIT;
  return std::min<int64_t>(s, SUM_MAX_SPLITS);
}

struct SumParams {
  const void* x; int64_t x_sb, x_st;
  int B, T, D, C;
  int seg_tokens; const int32_t* spans; int n_seg; int splits;
  const float2* factors; int nt, row_tokens, n_rows;
  float* ws;
};

__device__ __forceinline__ void segment_bounds(const SumParams& p, int seg, int& s0, int& s1) {
  if (p.spans) {
    s0 = p.spans[2 * seg];
    s1 = p.spans[2 * seg + 1];
  } else {
    s0 = seg * p.seg_tokens;
    s1 = s0 + p.seg_tokens;
  }
  s0 = max(s0, 0);
  s1 = min(s1, p.T);
  if (s1 < s0) s1 = s0;
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256) summary_partial_kernel(SumParams p) {
  const int seg = blockIdx.x / p.splits, split = blockIdx.x % p.splits;
  const int b = blockIdx.z;
  const int c0 = (blockIdx.y * blockDim.x + threadIdx.x) * VEC;
  if (c0 >= p.C) return;
  int s0, s1;
  segment_bounds(p, seg, s0, s1);
  const int per = (s1 - s0 + p.splits - 1) / p.splits;
  const int ts = s0 + split * per, te = min(ts + per, s1);
  const int d0 = c0 % p.D;  // VEC divides D: the run stays inside one head
  const bool band = p.factors != nullptr && d0 < 2 * p.nt;
  const T* base = (const T*)p.x + (int64_t)b * p.x_sb + c0;

  // The de-rope factor row of a token is its frame (t / row_tokens). The factors of this thread's
  // band pairs are held in registers and reloaded only when the frame changes, which a token run
  // inside one frame (a page of whole frames) never does: no per-token division or table load.
  constexpr int NP = VEC >= 2 ? VEC / 2 : 1;
  float2 w[NP];
  int row = -1, next = 0;  // current frame and the first token of the next one
  auto set_row = [&](int t) {
    row = min(t / p.row_tokens, p.n_rows - 1);
    next = row == p.n_rows - 1 ? 0x7fffffff : (row + 1) * p.row_tokens;
    const float2* frow = p.factors + (int64_t)row * p.nt;
#pragma unroll
    for (int e = 0; e < NP; ++e) {
      const int pr = (d0 >> 1) + e;
      w[e] = pr < p.nt ? frow[pr] : float2{1.f, 0.f};
    }
  };
  if (band && ts < te) set_row(ts);

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  constexpr int U = 8;  // tokens in flight per thread
  for (int t = ts; t < te; t += U) {
    float f[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int tt = t + u < te ? t + u : ts;
      load_vec<T, VEC>(base + (int64_t)tt * p.x_st, f[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t + u < te) {
        if constexpr (VEC >= 2) {
          if (band) {
            if (t + u >= next) set_row(t + u);
            // complex pairs in the temporal band times the factor, in fp32, rounded to T
#pragma unroll
            for (int e = 0; e < VEC; e += 2) {
              if (((d0 + e) >> 1) < p.nt) {
                const float2 wv = w[e >> 1];
                const float re = f[u][e] * wv.x - f[u][e + 1] * wv.y;
                const float im = f[u][e] * wv.y + f[u][e + 1] * wv.x;
                f[u][e] = round_to<T>(re);
                f[u][e + 1] = round_to<T>(im);
              }
            }
          }
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += f[u][e];
      }
    }
  }
  float* out = p.ws + (((int64_t)seg * p.B + b) * p.splits + split) * p.C + c0;
#pragma unroll
  for (int e = 0; e < VEC; ++e) out[e] = acc[e];
}

// Grid (n_seg, column groups of 256); with `normalize` a single column group covers the row so the
// norm can be formed in the block.
__global__ void __launch_bounds__(256) summary_reduce_kernel(SumParams p, float* out, int normalize) {
  __shared__ float red[4];
  const int seg = blockIdx.x;
  int s0, s1;
  segment_bounds(p, seg, s0, s1);
  const float len = (float)(s1 - s0);
  float sq = 0.f;
  const int c_begin = blockIdx.y * blockDim.x + threadIdx.x, c_step = blockDim.x * gridDim.y;
  for (int c = c_begin; c < p.C; c += c_step) {
    float tot = 0.f;
    for (int b = 0; b < p.B; ++b) {
      const float* w = p.ws + ((int64_t)seg * p.B + b) * p.splits * (int64_t)p.C + c;
      // the split partials are loaded 16 at a time (all in flight together) and added in split order
      float s = 0.f;
      int sp = 0;
      for (; sp + 16 <= p.splits; sp += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = w[(int64_t)(sp + j) * p.C];
#pragma unroll
        for (int j = 0; j < 16; ++j) s += v[j];
      }
      if (sp < p.splits) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = sp + j < p.splits ? w[(int64_t)(sp + j) * p.C] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (sp + j < p.splits) s += v[j];
      }
      tot += s / len;
    }
    const float v = tot / (float)p.B;
    out[(int64_t)seg * p.C + c] = v;
    sq += v * v;
  }
  if (!normalize) return;
  sq = wa_wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  const float norm = sqrtf(red[0] + red[1] + red[2] + red[3]);
  const float denom = fmaxf(norm, 1e-12f);
  for (int c = threadIdx.x; c < p.C; c += blockDim.x) out[(int64_t)seg * p.C + c] /= denom;
}

// =============================================================================================
// Score + top-k: one workgroup of 1024 threads. Keys are (order-preserving score bits, inverted
// page index), sorted descending with a bitonic network in LDS; key 0 marks masked / padding.
// =============================================================================================
struct TopkParams {
  const float* index; int64_t index_stride;
  const float* query;
  int n_pages, dim;
  float scale;
  const uint8_t* mask;
  int k;
  float* scores; int32_t* sel; float* sel_scores;
};

__global__ void __launch_bounds__(1024) score_topk_kernel(TopkParams p) {
  __shared__ uint64_t keys[WA_HKV_MAX_PAGES];
  __shared__ float sc[WA_HKV_MAX_PAGES];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int pg = w; pg < p.n_pages; pg += 16) {
    const float* row = p.index + (int64_t)pg * p.index_stride;
    float s = 0.f;
    for (int i = lane; i < p.dim; i += 64) s += row[i] * p.query[i];
    s = wa_wave_sum(s);
    if (p.scale > 0.f) s = s / p.scale;
    if (lane == 0) {
      sc[pg] = s;
      if (p.scores) p.scores[pg] = s;
      const uint32_t hi = isnan(s) ? 0xFFFFFFFFu : wa_float_key(s);
      const bool masked = p.mask != nullptr && p.mask[pg] != 0;
      keys[pg] = masked ? 0ull : (((uint64_t)hi << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)pg));
    }
  }
  int n2 = 1;
  while (n2 < p.n_pages) n2 <<= 1;
  for (int i = p.n_pages + tid; i < n2; i += 1024) keys[i] = 0ull;
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < n2 / 2; i += 1024) {
        const int lo = 2 * stride * (i / stride) + (i % stride), hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = keys[lo], c = keys[hi];
        if ((a < c) == desc) {
          keys[lo] = c;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < p.k; i += 1024) {
    const uint64_t key = i < n2 ? keys[i] : 0ull;
    if (key == 0ull) {
      p.sel[i] = -1;
      p.sel_scores[i] = -INFINITY;
    } else {
      const int pg = (int)(0xFFFFFFFFu - (uint32_t)key);
      p.sel[i] = pg;
      p.sel_scores[i] = sc[pg];
    }
  }
}

// =============================================================================================
// Rerope: one thread per VEC-channel run of one (b, t, h); in place only the band runs exist.
// =============================================================================================
struct RopeParams {
  const void* src; int64_t s_sb, s_st, s_sh;
  void* dst; int64_t d_sb, d_st, d_sh;
  int B, t0, ntok, H, D;
  const float2* factors; int nt, n_rows;
  const int32_t* rows; int row_tokens;
  int runs;  // VEC runs per head processed
};

template <typename T, int VEC>
__global__ void __launch_bounds__(256) rerope_kernel(RopeParams p) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.ntok * p.H * p.runs;
  if (gid >= total) return;
  int64_t r = gid;
  const int run = (int)(r % p.runs);
  r /= p.runs;
  const int h = (int)(r % p.H);
  r /= p.H;
  const int tl = (int)(r % p.ntok);
  const int b = (int)(r / p.ntok);
  const int64_t t = p.t0 + tl;
  const int d0 = run * VEC;
  float f[VEC];
  load_vec<T, VEC>((const T*)p.src + (int64_t)b * p.s_sb + t * p.s_st + (int64_t)h * p.s_sh + d0, f);
  if (d0 < 2 * p.nt) {
    int row = p.rows ? p.rows[tl] : tl / p.row_tokens;
    row = min(max(row, 0), p.n_rows - 1);
    rotate_band<T, VEC>(f, d0, p.factors + (int64_t)row * p.nt, p.nt);
  }
  store_vec<T, VEC>((T*)p.dst + (int64_t)b * p.d_sb + t * p.d_st + (int64_t)h * p.d_sh + d0, f);
}

// =============================================================================================
// Gather + rotate: key pages read straight from pinned host memory (through the device mapping)
// into the cache, the temporal band rotated on the way; one factor row per page. Work item = one
// VEC-channel run of one (b, token, head); up to GR_MAX pages per launch. The grid is small and
// fixed (GR_BLOCKS workgroups striding over the items, each thread with GR_UNROLL host reads in
// flight before it rotates and stores any): the host link stays saturated while the install holds
// only a few CUs, so attention kernels running beside it keep the rest. (One thread per item made
// ~9,400 workgroups per cfg 3 layer, each waiting on host reads and together holding every CU.)
// =============================================================================================
constexpr int GR_MAX = 32;
constexpr int GR_BLOCKS = 128;
constexpr int GR_UNROLL = 8;
struct GRPage {
  const void* src; int64_t s_sb, s_st, s_sh;
  int tokens, dst_token;
  int64_t start;  // first thread id of the page
};
struct GatherRotParams {
  GRPage pg[GR_MAX];
  int n;
  void* dst; int64_t d_sb, d_st, d_sh;
  int B, H, D, runs;
  const float2* factors; int nt;
  int64_t total;
};

template <typename T, int VEC>
__global__ void __launch_bounds__(256) gather_rotate_kernel(GatherRotParams p) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t base = (int64_t)blockIdx.x * 256 + threadIdx.x; base < p.total; base += stride * GR_UNROLL) {
    float f[GR_UNROLL][VEC];
    int64_t dst[GR_UNROLL];
    int page[GR_UNROLL], d0[GR_UNROLL];
#pragma unroll
    for (int u = 0; u < GR_UNROLL; ++u) {
      const int64_t gid = base + u * stride;
      page[u] = -1;
      if (gid >= p.total) continue;
      int j = 0;
      while (j + 1 < p.n && gid >= p.pg[j + 1].start) ++j;
      const GRPage& g = p.pg[j];
      int64_t r = gid - g.start;
      const int run = (int)(r % p.runs);
      r /= p.runs;
      const int h = (int)(r % p.H);
      r /= p.H;
      const int tl = (int)(r % g.tokens);
      const int b = (int)(r / g.tokens);
      page[u] = j;
      d0[u] = run * VEC;
      dst[u] = (int64_t)b * p.d_sb + (int64_t)(g.dst_token + tl) * p.d_st + (int64_t)h * p.d_sh + d0[u];
      load_vec<T, VEC>((const T*)g.src + (int64_t)b * g.s_sb + (int64_t)tl * g.s_st + (int64_t)h * g.s_sh + d0[u], f[u]);
    }
#pragma unroll
    for (int u = 0; u < GR_UNROLL; ++u) {
      if (page[u] < 0) continue;
      if (p.factors && d0[u] < 2 * p.nt) rotate_band<T, VEC>(f[u], d0[u], p.factors + (int64_t)page[u] * p.nt, p.nt);
      store_vec<T, VEC>((T*)p.dst + dst[u], f[u]);
    }
  }
}

bool fits_int(int64_t v) { return v >= 0 && v <= (int64_t)0x7fffffff; }

int hkv_copies(const wa_hkv_copy* c, int64_t n, hipMemcpyKind kind, void* stream, void* done, const char* what) {
  WA_CHECK_ARG(n >= 0 && (n == 0 || c != nullptr), "%s: bad copy list", what);
  hipStream_t s = (hipStream_t)stream;
  for (int64_t i = 0; i < n; ++i) {
    const wa_hkv_copy& k = c[i];
    WA_CHECK_ARG(k.src && k.dst && k.width > 0 && k.rows >= 1, "%s: copy %lld is empty or null", what, (long long)i);
    WA_CHECK_ARG(k.rows == 1 || (k.src_pitch >= k.width && k.dst_pitch >= k.width),
                 "%s: copy %lld has a pitch below its width", what, (long long)i);
    const void* host = kind == hipMemcpyHostToDevice ? k.src : (const void*)k.dst;
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, host);
    if (e != hipSuccess) (void)hipGetLastError();
    WA_CHECK_ARG(e == hipSuccess && attr.type == hipMemoryTypeHost,
                 "%s: copy %lld: the host buffer is not pinned (allocate it with hipHostMalloc)", what,
                 (long long)i);
    if (k.rows == 1)
      WA_CHECK_HIP(hipMemcpyAsync(k.dst, k.src, (size_t)k.width, kind, s));
    else
      WA_CHECK_HIP(hipMemcpy2DAsync(k.dst, (size_t)k.dst_pitch, k.src, (size_t)k.src_pitch, (size_t)k.width,
                                    (size_t)k.rows, kind, s));
  }
  if (done) WA_CHECK_HIP(hipEventRecord((hipEvent_t)done, s));
  return WA_OK;
}

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================
extern "C" int64_t wa_hkv_summary_workspace_bytes(int64_t B, int64_t n_seg, int64_t C, int64_t max_seg_tokens) {
  if (B <= 0 || n_seg <= 0 || C <= 0) return 0;
  return B * n_seg * C * summary_splits(max_seg_tokens) * (int64_t)sizeof(float);
}

extern "C" int wa_hkv_page_summary(const wa_hkv_summary_args* a, void* stream) {
  WA_CHECK_ARG(a && a->x && a->out && a->workspace, "wa_hkv_page_summary: null argument");
  WA_CHECK_ARG(a->x_dtype == WA_BF16 || a->x_dtype == WA_F32, "wa_hkv_page_summary: x must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 1 && a->T >= 0 && a->H >= 1 && a->D >= 1 && (a->factors == nullptr || a->D % 2 == 0),
               "wa_hkv_page_summary: bad shape B=%lld T=%lld H=%lld D=%lld", (long long)a->B, (long long)a->T,
               (long long)a->H, (long long)a->D);
  WA_CHECK_ARG(a->n_seg >= 1 && a->n_seg <= 65535 * 64, "wa_hkv_page_summary: n_seg out of range");
  WA_CHECK_ARG(a->spans != nullptr || a->seg_tokens >= 1, "wa_hkv_page_summary: need spans or seg_tokens >= 1");
  WA_CHECK_ARG(a->max_seg_tokens >= 1, "wa_hkv_page_summary: max_seg_tokens must be >= 1");
  WA_CHECK_ARG(a->spans != nullptr || a->seg_tokens <= a->max_seg_tokens,
               "wa_hkv_page_summary: seg_tokens exceeds max_seg_tokens");
  if (a->factors) {
    WA_CHECK_ARG(a->n_temporal >= 1 && 2 * a->n_temporal <= a->D && a->row_tokens >= 1 && a->n_rows >= 1,
                 "wa_hkv_page_summary: bad de-rope table (n_temporal=%lld row_tokens=%lld n_rows=%lld)",
                 (long long)a->n_temporal, (long long)a->row_tokens, (long long)a->n_rows);
  }
  const int64_t C = a->H * a->D;
  WA_CHECK_ARG(fits_int(C) && fits_int(a->T), "wa_hkv_page_summary: sizes exceed int32");
  const int64_t splits = summary_splits(a->max_seg_tokens);
  const bool vec8 = a->D % 8 == 0 && a->x_sb % 8 == 0 && a->x_st % 8 == 0 && wa_aligned16(a->x);
  const int vec = vec8 ? 8 : (a->D % 2 == 0 ? 2 : 1);
  const int64_t lanes = (C + vec - 1) / vec;
  const int threads = (int)std::min<int64_t>(256, ((lanes + 63) / 64) * 64);
  const int64_t col_groups = (lanes + threads - 1) / threads;
  WA_CHECK_ARG(a->n_seg * splits <= 0x7fffffff && col_groups <= 65535 && a->B <= 65535,
               "wa_hkv_page_summary: grid too large");

  SumParams p{a->x, a->x_sb, a->x_st, (int)a->B, (int)a->T, (int)a->D, (int)C,
              (int)std::min<int64_t>(a->seg_tokens, 0x7fffffff), a->spans, (int)a->n_seg, (int)splits,
              (const float2*)a->factors, (int)a->n_temporal, (int)std::max<int64_t>(a->row_tokens, 1),
              (int)std::max<int64_t>(a->n_rows, 1), (float*)a->workspace};
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(a->n_seg * splits), (unsigned)col_groups, (unsigned)a->B);
  if (a->x_dtype == WA_BF16) {
    if (vec == 8) summary_partial_kernel<bf16_t, 8><<<grid, threads, 0, s>>>(p);
    else if (vec == 2) summary_partial_kernel<bf16_t, 2><<<grid, threads, 0, s>>>(p);
    else summary_partial_kernel<bf16_t, 1><<<grid, threads, 0, s>>>(p);
  } else {
    if (vec == 8) summary_partial_kernel<float, 8><<<grid, threads, 0, s>>>(p);
    else if (vec == 2) summary_partial_kernel<float, 2><<<grid, threads, 0, s>>>(p);
    else summary_partial_kernel<float, 1><<<grid, threads, 0, s>>>(p);
  }
  int rc = wa_launch_status("summary_partial_kernel");
  if (rc) return rc;
  const unsigned red_groups = a->normalize ? 1u : (unsigned)std::min<int64_t>((C + 255) / 256, 65535);
  summary_reduce_kernel<<<dim3((unsigned)a->n_seg, red_groups), 256, 0, s>>>(p, a->out, a->normalize ? 1 : 0);
  return wa_launch_status("summary_reduce_kernel");
}

extern "C" int wa_hkv_score_topk(const wa_hkv_topk_args* a, void* stream) {
  WA_CHECK_ARG(a && a->index && a->query && a->sel && a->sel_scores, "wa_hkv_score_topk: null argument");
  WA_CHECK_ARG(a->n_pages >= 1 && a->n_pages <= WA_HKV_MAX_PAGES,
               "wa_hkv_score_topk: n_pages=%lld outside [1, %d]", (long long)a->n_pages, WA_HKV_MAX_PAGES);
  WA_CHECK_ARG(a->dim >= 1 && fits_int(a->dim) && a->index_stride >= a->dim, "wa_hkv_score_topk: bad dim/stride");
  WA_CHECK_ARG(a->k >= 1 && a->k <= a->n_pages, "wa_hkv_score_topk: k=%lld outside [1, n_pages]", (long long)a->k);
  TopkParams p{a->index, a->index_stride, a->query, (int)a->n_pages, (int)a->dim, a->scale, a->mask,
               (int)a->k, a->scores, a->sel, a->sel_scores};
  score_topk_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(p);
  return wa_launch_status("score_topk_kernel");
}

extern "C" int wa_rerope(const wa_rerope_args* a, void* stream) {
  WA_CHECK_ARG(a && a->src && a->dst && a->factors, "wa_rerope: null argument");
  WA_CHECK_ARG(a->dtype == WA_BF16 || a->dtype == WA_F32, "wa_rerope: dtype must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 1 && a->H >= 1 && a->D >= 2 && a->D % 2 == 0 && a->t0 >= 0 && a->t1 >= a->t0,
               "wa_rerope: bad shape");
  WA_CHECK_ARG(a->n_temporal >= 1 && 2 * a->n_temporal <= a->D && a->n_rows >= 1,
               "wa_rerope: bad factor table (n_temporal=%lld n_rows=%lld)", (long long)a->n_temporal,
               (long long)a->n_rows);
  WA_CHECK_ARG(a->rows != nullptr || a->row_tokens >= 1, "wa_rerope: need rows or row_tokens >= 1");
  const int64_t ntok = a->t1 - a->t0;
  if (ntok == 0) return WA_OK;
  WA_CHECK_ARG(fits_int(ntok) && fits_int(a->t1) && fits_int(a->D) && fits_int(a->H) && fits_int(a->B),
               "wa_rerope: sizes exceed int32");
  const bool inplace = a->src == a->dst;
  const bool vec8 = a->D % 8 == 0 && a->s_sb % 8 == 0 && a->s_st % 8 == 0 && a->s_sh % 8 == 0 &&
                    a->d_sb % 8 == 0 && a->d_st % 8 == 0 && a->d_sh % 8 == 0 &&
                    wa_aligned16(a->src) && wa_aligned16(a->dst);
  const int vec = vec8 ? 8 : 2;
  const int64_t runs = inplace ? (2 * a->n_temporal + vec - 1) / vec : a->D / vec;
  const int64_t total = a->B * ntok * a->H * runs;
  const int64_t blocks = (total + 255) / 256;
  WA_CHECK_ARG(blocks <= 0x7fffffff, "wa_rerope: grid too large");
  RopeParams p{a->src, a->s_sb, a->s_st, a->s_sh, a->dst, a->d_sb, a->d_st, a->d_sh,
               (int)a->B, (int)a->t0, (int)ntok, (int)a->H, (int)a->D,
               (const float2*)a->factors, (int)a->n_temporal, (int)std::min<int64_t>(a->n_rows, 0x7fffffff),
               a->rows, (int)std::max<int64_t>(std::min<int64_t>(a->row_tokens, 0x7fffffff), 1), (int)runs};
  hipStream_t s = (hipStream_t)stream;
  if (a->dtype == WA_BF16) {
    if (vec8) rerope_kernel<bf16_t, 8><<<(unsigned)blocks, 256, 0, s>>>(p);
    else rerope_kernel<bf16_t, 2><<<(unsigned)blocks, 256, 0, s>>>(p);
  } else {
    if (vec8) rerope_kernel<float, 8><<<(unsigned)blocks, 256, 0, s>>>(p);
    else rerope_kernel<float, 2><<<(unsigned)blocks, 256, 0, s>>>(p);
  }
  return wa_launch_status("rerope_kernel");
}

extern "C" int wa_hkv_gather_rotate(const wa_hkv_gather_rotate_args* a, void* stream) {
  WA_CHECK_ARG(a && a->dst && (a->n_pages == 0 || a->pages), "wa_hkv_gather_rotate: null argument");
  WA_CHECK_ARG(a->dtype == WA_BF16 || a->dtype == WA_F32, "wa_hkv_gather_rotate: dtype must be bf16 or fp32");
  WA_CHECK_ARG(a->B >= 1 && a->H >= 1 && a->D >= 2 && a->D % 2 == 0 && a->cap >= 1 && a->n_pages >= 0,
               "wa_hkv_gather_rotate: bad shape");
  WA_CHECK_ARG(!a->factors || (a->n_temporal >= 1 && 2 * a->n_temporal <= a->D),
               "wa_hkv_gather_rotate: bad factor table (n_temporal=%lld)", (long long)a->n_temporal);
  WA_CHECK_ARG(fits_int(a->B * a->cap) && fits_int(a->H) && fits_int(a->D), "wa_hkv_gather_rotate: sizes exceed int32");
  const bool vec_dst = a->D % 8 == 0 && a->d_sb % 8 == 0 && a->d_st % 8 == 0 && a->d_sh % 8 == 0 && wa_aligned16(a->dst);
  bool vec8 = vec_dst;
  // every page: pinned host memory with a device mapping, inside the cache
  std::vector<const void*> dev_src((size_t)a->n_pages);
  for (int64_t i = 0; i < a->n_pages; ++i) {
    const wa_hkv_page& g = a->pages[i];
    WA_CHECK_ARG(g.src && g.tokens >= 0 && g.dst_token >= 0 && g.dst_token + g.tokens <= a->cap,
                 "wa_hkv_gather_rotate: page %lld: tokens [%lld, %lld) outside a cache of %lld", (long long)i,
                 (long long)g.dst_token, (long long)(g.dst_token + g.tokens), (long long)a->cap);
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, g.src);
    if (e != hipSuccess) (void)hipGetLastError();
    WA_CHECK_ARG(e == hipSuccess && attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr,
                 "wa_hkv_gather_rotate: page %lld is not pinned host memory with a device mapping", (long long)i);
    dev_src[(size_t)i] = attr.devicePointer;
    vec8 = vec8 && g.s_sb % 8 == 0 && g.s_st % 8 == 0 && g.s_sh % 8 == 0 && wa_aligned16(attr.devicePointer);
  }
  const int vec = vec8 ? 8 : 2;
  const int64_t runs = a->D / vec;
  hipStream_t s = (hipStream_t)stream;
  for (int64_t p0 = 0; p0 < a->n_pages; p0 += GR_MAX) {
    GatherRotParams p{};
    p.n = 0;
    int64_t total = 0;
    for (int64_t i = p0; i < std::min<int64_t>(a->n_pages, p0 + GR_MAX); ++i) {
      const wa_hkv_page& g = a->pages[i];
      if (g.tokens == 0) continue;
      p.pg[p.n] = GRPage{dev_src[(size_t)i], g.s_sb, g.s_st, g.s_sh, (int)g.tokens, (int)g.dst_token, total};
      total += a->B * g.tokens * a->H * runs;
      ++p.n;
    }
    if (p.n == 0) continue;
    p.dst = a->dst; p.d_sb = a->d_sb; p.d_st = a->d_st; p.d_sh = a->d_sh;
    p.B = (int)a->B; p.H = (int)a->H; p.D = (int)a->D; p.runs = (int)runs;
    p.factors = (const float2*)a->factors;
    p.nt = (int)a->n_temporal;
    p.total = total;
    // factor row j of the launch is the caller's row p0 + j, so no page may be skipped then
    if (a->factors) {
      WA_CHECK_ARG(p.n == std::min<int64_t>(a->n_pages, p0 + GR_MAX) - p0,
                   "wa_hkv_gather_rotate: empty pages are not allowed with a factor table");
      p.factors = (const float2*)a->factors + p0 * a->n_temporal;
    }
    const int64_t blocks = std::min<int64_t>(GR_BLOCKS, (total + 256 * GR_UNROLL - 1) / (256 * GR_UNROLL));
    if (a->dtype == WA_BF16) {
      if (vec8) gather_rotate_kernel<bf16_t, 8><<<(unsigned)blocks, 256, 0, s>>>(p);
      else gather_rotate_kernel<bf16_t, 2><<<(unsigned)blocks, 256, 0, s>>>(p);
    } else {
      if (vec8) gather_rotate_kernel<float, 8><<<(unsigned)blocks, 256, 0, s>>>(p);
      else gather_rotate_kernel<float, 2><<<(unsigned)blocks, 256, 0, s>>>(p);
    }
    const int rc = wa_launch_status("gather_rotate_kernel");
    if (rc != WA_OK) return rc;
  }
  return WA_OK;
}

extern "C" int wa_hkv_gather_async(const wa_hkv_copy* copies, int64_t n, void* stream, void* done) {
  return hkv_copies(copies, n, hipMemcpyHostToDevice, stream, done, "wa_hkv_gather_async");
}

extern "C" int wa_hkv_store_async(const wa_hkv_copy* copies, int64_t n, void* stream, void* done) {
  return hkv_copies(copies, n, hipMemcpyDeviceToHost, stream, done, "wa_hkv_store_async");
}
