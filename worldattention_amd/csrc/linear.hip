// Low-rank linear branch of the reference (wan/modules/hsa/attention.py:64-118) for gfx950:
//  * compress_kv — low-rank sequence projection per segment (attention.py:64-110); the softmax
//    over the compressed keys then runs in the block-sparse kernel as dense attention;
//  * its backward (dx and the projection's gradient) for training in the reference's head mode.
// The contraction runs on v_mfma_f32_32x32x16_bf16 with fp32 accumulation; the token-axis
// operand is staged through LDS transposed ([channel][token]).
// The north-star elu(x)+1 linear branch lives in elu1.hip.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "tile.h"

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
  int64_t x_slab;   // bytes of one (batch, head) x slab: first row to the last row's end
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
// compress_kv for bf16 x with 16-byte aligned rows, as out^T[d, r] = sum_t x^T[d, t] E^T[t, r]:
// the segment's x rows stream global -> LDS in 64-token tiles (direct-to-LDS loads, a 4-stage
// ring, three tiles in flight; inline-assembly loads that the kernel orders itself, so the
// compiler adds no waits of its own), each with the 32 x 64 slice of E it needs; wave w takes the A
// operand of its 32 channels by transpose reads of the row-major x tile and the B operand (lane =
// row r of E, 8 consecutive tokens) by one 16-byte read of the E slice. Rows of E past this
// segment's rank and rows of x past the tensor's end read zeros (buffer range); tokens past the
// segment's end get zero weights in its last tile. One workgroup per (segment, head, batch): the
// compress of a tensor streams at HBM speed instead of one memory round trip per 64 tokens.
// =============================================================================================
template <int D>
__global__ void __launch_bounds__(2 * D) compress_stream_kernel(CompressParams p) {
  constexpr int NW = D / 32, TILE = 64 * D, SS = TILE + 32 * 64;  // stage: x tile, then E slice
  constexpr int CPR = D / 8, RPI = 64 / CPR, NI = 64 / (RPI * NW);  // x tile: NI loads per wave
  constexpr int EI = 4 / NW;                                         // E slice: EI loads per wave
  __shared__ __attribute__((aligned(1024))) bf16_t st0[SS];
  __shared__ __attribute__((aligned(1024))) bf16_t st1[SS];
  __shared__ __attribute__((aligned(1024))) bf16_t st2[SS];
  __shared__ __attribute__((aligned(1024))) bf16_t st3[SS];
  const int sidx = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int start = sidx * p.seg;
  const int seg_len = min(p.seg, p.L - start);
  const int rank = min(p.proj_rank, (seg_len + p.block - 1) / p.block);
  const int row0 = sidx * min(p.proj_rank, (p.seg + p.block - 1) / p.block);
  const int nt = (seg_len + 63) / 64;

  // x tile i = segment tokens 64 i .. 64 i + 63: lane L of wave instruction k writes row
  // (k NW + w) RPI + L / CPR, chunk slot L % CPR (dual swizzle)
  const char* xbase = (const char*)p.x + ((int64_t)b * p.x_sb + (int64_t)h * p.x_sh) * 2;
  int xoff[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int row = (k * NW + w) * RPI + lane / CPR, pos = lane % CPR;
    xoff[k] = (int)(row * p.x_st * 2) + (pos ^ dual_swizzle<D>(row)) * 16;
  }
  // E slice of tile i: rank rows 0..31 x tokens 64 i .. +63 (128 bytes a row); lane L of wave
  // instruction k writes row (k NW + w) 8 + L / 8, chunk slot L % 8 holding chunk slot ^ (row & 7)
  int eoff[EI];
#pragma unroll
  for (int k = 0; k < EI; ++k) {
    const int row = (k * NW + w) * 8 + lane / 8, pos = lane % 8;
    eoff[k] = row < rank ? row * p.proj_len * 2 + ((pos ^ (row & 7)) * 16) : 0x7fff0000;  // past the range: 0
  }
  auto issue = [&](bf16_t* stage, int i) {
    if (i >= nt) return;  // uniform
    const int64_t o = (int64_t)(start + 64 * i) * p.x_st * 2;
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(xbase + o), (short)0, (int)(p.x_slab - o), WA_BUF_DWORD3);
#pragma unroll
    for (int k = 0; k < NI; ++k) lds_dma16(xrs, stage + (k * NW + w) * RPI * D, xoff[k]);
    const __amdgpu_buffer_rsrc_t ers = __builtin_amdgcn_make_buffer_rsrc((void*)((const char*)p.proj + 128 * i), (short)0,
                                                                         p.proj_rank * p.proj_len * 2 - 128 * i, WA_BUF_DWORD3);
#pragma unroll
    for (int k = 0; k < EI; ++k) lds_dma16(ers, stage + TILE + (k * NW + w) * 512, eoff[k]);
  };
  issue(st0, 0);
  issue(st1, 1);
  issue(st2, 2);
  f32x16 acc = f32x16{};
  // tile i computes on stage i % 4; every tile issues the same NI + EI loads per wave, so tile i has
  // landed once at most that many per later tile remain in flight
  auto step = [&](bf16_t* stage, bf16_t* refill, int i) {
    const int ahead = min(2, nt - 1 - i);
    if (ahead >= 2) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * (NI + EI)) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NI + EI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    bf16x8 ef[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) ef[c] = *(const bf16x8*)(stage + TILE + l32 * 64 + (((2 * c + g) ^ (l32 & 7)) * 8));
    if (64 * i + 64 > seg_len) {  // uniform: the segment's partial last tile
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ef[c][e] = 64 * i + 16 * c + 8 * g + e < seg_len ? ef[c][e] : (bf16_t)0.f;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) acc = wa_mfma32(tile_tr8n<D>(stage, c, 32 * w, lane), ef[c], acc);
    // the stage of tile i - 1, which every wave had read before the barrier above (issued after
    // this tile's reads, so that no read of this stage waits for it)
    issue(refill, i + 3);
  };
  for (int i = 0; i < nt; i += 4) {
    step(st0, st3, i);
    if (i + 1 < nt) step(st1, st0, i + 1);
    if (i + 2 < nt) step(st2, st1, i + 2);
    if (i + 3 < nt) step(st3, st2, i + 3);
  }
  // lane l32 holds rank row r = l32, channels d = 32 w + 8 (i / 4) + 4 g + i % 4
  if (l32 >= rank) return;
  const int64_t o0 = (int64_t)b * p.o_sb + (int64_t)(row0 + l32) * p.o_st + (int64_t)h * p.o_sh + 32 * w + 4 * g;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
#pragma unroll
    for (int i = 0; i < 4; ++i) wa_store_f(p.out, o0 + 8 * rq + i, acc[rq * 4 + i], p.o_dtype);
  }
}

// =============================================================================================
// compress_kv backward. For segment s (tokens start .. start + n, rows row0 .. row0 + r of the
// compressed output, row0 = s * r_full): dx[start + t] = sum_j E[j, t] dout[row0 + j] and the
// segment's share of dE[j, t] = sum_{b, h, d} dout[b, row0 + j, h, d] x[b, start + t, h, d].
// fp32 arithmetic throughout; E is the projection's stored value (bf16 widened exactly).
// =============================================================================================
struct CompressBwdParams {
  const float* dout; int64_t d_sb, d_st, d_sh;
  const void* x; int64_t x_sb, x_st, x_sh; int x_dtype;
  const void* proj; int proj_dtype; int R, P;
  int B, L, H, D, seg, block, n_first, r_full, n_seg;
  float* dx; int64_t dx_sb, dx_st, dx_sh; int dx_acc;
  float* dproj; int dproj_acc;
  float* part;  // [n_seg][r_full][n_first]
};

__device__ __forceinline__ float proj_at(const CompressBwdParams& p, int j, int t) {
  const int64_t off = (int64_t)j * p.P + t;
  return p.proj_dtype == WA_BF16 ? (float)((const bf16_t*)p.proj)[off] : ((const float*)p.proj)[off];
}

// dx: one workgroup per (16-token tile of a segment, 128 float4 columns of (head, channel), batch);
// a thread keeps its column of the segment's dout rows 16 at a time in registers and the matching
// 16 x 16 block of E in LDS, and sums over j in increasing order.
constexpr int kDxTokens = 16, kDxRows = 16, kDxThreads = 128;
__global__ void __launch_bounds__(kDxThreads) compress_bwd_dx_kernel(CompressBwdParams p) {
  __shared__ float es[kDxRows][kDxTokens];
  const int tps = (p.n_first + kDxTokens - 1) / kDxTokens;
  const int s = blockIdx.x / tps, t0 = (blockIdx.x % tps) * kDxTokens, b = blockIdx.z;
  const int start = s * p.seg, n = min(p.seg, p.L - start);
  if (t0 >= n) return;  // uniform
  const int r = min(p.R, (n + p.block - 1) / p.block), row0 = s * p.r_full;
  const int tid = threadIdx.x;
  const int c = blockIdx.y * kDxThreads + tid;  // float4 column
  const bool active = c < p.H * p.D / 4;
  const int h = active ? c * 4 / p.D : 0, d = active ? c * 4 % p.D : 0;
  const float* gcol = p.dout + (int64_t)b * p.d_sb + (int64_t)h * p.d_sh + d;
  f32x4 acc[kDxTokens];
#pragma unroll
  for (int i = 0; i < kDxTokens; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < r; j0 += kDxRows) {
    __syncthreads();  // the previous block of E has been read
    for (int i = tid; i < kDxRows * kDxTokens; i += kDxThreads) {
      const int jj = i / kDxTokens, tl = i % kDxTokens, j = j0 + jj, t = t0 + tl;
      es[jj][tl] = j < r && t < n ? proj_at(p, j, t) : 0.f;
    }
    f32x4 g[kDxRows];
#pragma unroll
    for (int jj = 0; jj < kDxRows; ++jj)
      g[jj] = active && j0 + jj < r ? *(const f32x4*)(gcol + (int64_t)(row0 + j0 + jj) * p.d_st)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();
#pragma unroll
    for (int tl = 0; tl < kDxTokens; ++tl) {
#pragma unroll
      for (int jj = 0; jj < kDxRows; ++jj) {
        const float e = es[jj][tl];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[tl][q] = fmaf(e, g[jj][q], acc[tl][q]);
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int tl = 0; tl < kDxTokens; ++tl) {
    const int t = t0 + tl;
    if (t >= n) break;
    f32x4* dst = (f32x4*)(p.dx + (int64_t)b * p.dx_sb + (int64_t)(start + t) * p.dx_st + (int64_t)h * p.dx_sh + d);
    *dst = p.dx_acc ? *dst + acc[tl] : acc[tl];
  }
}

// dE share of one segment: one workgroup of 4 waves per (64-token tile, segment); lane = token,
// wave w sums heads w, w + 4, ... of every batch for all r rows, then the four waves' sums are added
// in wave order through LDS into the segment's partial.
template <int RMAX>
__global__ void __launch_bounds__(256) compress_bwd_dproj_kernel(CompressBwdParams p) {
  __shared__ float red[4][16][64];
  const int s = blockIdx.y, t0 = blockIdx.x * 64;
  const int start = s * p.seg, n = min(p.seg, p.L - start);
  if (t0 >= n) return;  // uniform
  const int r = min(p.R, (n + p.block - 1) / p.block), row0 = s * p.r_full;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int t = t0 + lane;
  const bool ok = t < n;
  float acc[RMAX];
#pragma unroll
  for (int j = 0; j < RMAX; ++j) acc[j] = 0.f;
  for (int b = 0; b < p.B; ++b) {
    for (int h = w; h < p.H; h += 4) {
      const int64_t xo = (int64_t)b * p.x_sb + (int64_t)(start + (ok ? t : 0)) * p.x_st + (int64_t)h * p.x_sh;
      const float* grow = p.dout + (int64_t)b * p.d_sb + (int64_t)row0 * p.d_st + (int64_t)h * p.d_sh;
      for (int d0 = 0; d0 < p.D; d0 += 8) {
        float xf[8];
        if (p.x_dtype == WA_BF16) {
          const bf16x8 v = *(const bf16x8*)((const bf16_t*)p.x + xo + d0);
#pragma unroll
          for (int e = 0; e < 8; ++e) xf[e] = ok ? (float)v[e] : 0.f;
        } else {
          const f32x4 v0 = *(const f32x4*)((const float*)p.x + xo + d0);
          const f32x4 v1 = *(const f32x4*)((const float*)p.x + xo + d0 + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xf[e] = ok ? v0[e] : 0.f;
            xf[4 + e] = ok ? v1[e] : 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < RMAX; ++j) {
          if (j >= r) break;
          const f32x4 g0 = *(const f32x4*)(grow + (int64_t)j * p.d_st + d0);
          const f32x4 g1 = *(const f32x4*)(grow + (int64_t)j * p.d_st + d0 + 4);
          float a = acc[j];
#pragma unroll
          for (int e = 0; e < 4; ++e) a = fmaf(xf[e], g0[e], a);
#pragma unroll
          for (int e = 0; e < 4; ++e) a = fmaf(xf[4 + e], g1[e], a);
          acc[j] = a;
        }
      }
    }
  }
  float* part = p.part + (int64_t)s * p.r_full * p.n_first;
#pragma unroll
  for (int j0 = 0; j0 < RMAX; j0 += 16) {
    if (j0 >= r) break;
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) red[w][jj][lane] = acc[j0 + jj < RMAX ? j0 + jj : 0];
    __syncthreads();
    // wave q writes rows j0 + q, j0 + q + 4, ...: the sum over waves 0..3 in order
    for (int jj = w; jj < 16; jj += 4) {
      const int j = j0 + jj;
      if (j < r && ok)
        part[(int64_t)j * p.n_first + t] = ((red[0][jj][lane] + red[1][jj][lane]) + red[2][jj][lane]) + red[3][jj][lane];
    }
  }
}

// dproj[j, t] (+)= sum over segments, in segment order, of the partials that cover (j, t); every
// entry of the [R, P] matrix is visited, so in write mode untouched entries become zero.
__global__ void __launch_bounds__(256) compress_bwd_reduce_kernel(CompressBwdParams p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.R * p.P) return;
  const int j = (int)(i / p.P), t = (int)(i % p.P);
  float sum = 0.f;
  if (j < p.r_full && t < p.n_first) {
    for (int s = 0; s < p.n_seg; ++s) {
      const int n = min(p.seg, p.L - s * p.seg);
      const int r = min(p.R, (n + p.block - 1) / p.block);
      if (j < r && t < n) sum += p.part[((int64_t)s * p.r_full + j) * p.n_first + t];
    }
  }
  p.dproj[i] = p.dproj_acc ? p.dproj[i] + sum : sum;
}

}  // namespace

extern "C" int64_t wa_compress_kv_bwd_workspace_bytes(int64_t L, int64_t proj_rank, int64_t segment_len,
                                                      int64_t block_size) {
  if (L <= 0 || proj_rank <= 0 || segment_len <= 0 || block_size <= 0) return 0;
  const int64_t n_first = segment_len < L ? segment_len : L;
  const int64_t r_full = std::min(proj_rank, (n_first + block_size - 1) / block_size);
  const int64_t n_seg = (L + segment_len - 1) / segment_len;
  return n_seg * r_full * n_first * 4;
}

extern "C" int wa_compress_kv_bwd(const wa_compress_bwd_args* a, void* stream) {
  WA_CHECK_ARG(a && a->dout && a->x && a->proj, "wa_compress_kv_bwd: null argument");
  WA_CHECK_ARG(a->dproj == nullptr || a->workspace != nullptr, "wa_compress_kv_bwd: dproj needs the workspace");
  WA_CHECK_ARG(a->D == 32 || a->D == 64 || a->D == 128, "wa_compress_kv_bwd: head dim %lld not in {32, 64, 128}",
               (long long)a->D);
  WA_CHECK_ARG(a->x_dtype == WA_F32 || a->x_dtype == WA_BF16, "wa_compress_kv_bwd: bad dtype");
  WA_CHECK_ARG(a->proj_dtype == WA_F32 || a->proj_dtype == WA_BF16, "wa_compress_kv_bwd: bad proj dtype");
  WA_CHECK_ARG(a->segment_len > 0 && a->block_size > 0 && a->L > 0 && a->B >= 0 && a->H > 0,
               "wa_compress_kv_bwd: bad sizes");
  WA_CHECK_ARG(a->proj_rank > 0 && a->proj_rank <= 128, "wa_compress_kv_bwd: projection rank must be in [1, 128]");
  const int64_t n_first = a->segment_len < a->L ? a->segment_len : a->L;
  WA_CHECK_ARG(n_first <= a->proj_len, "wa_compress_kv_bwd: segment length %lld exceeds projection length %lld",
               (long long)n_first, (long long)a->proj_len);
  // vector accesses: dout / dx by float4, x by 16 bytes (8 bf16 or 2 x 4 fp32)
  const int64_t xv = a->x_dtype == WA_BF16 ? 8 : 4;
  WA_CHECK_ARG(wa_aligned16(a->dout) && a->d_sb % 4 == 0 && a->d_st % 4 == 0 && a->d_sh % 4 == 0,
               "wa_compress_kv_bwd: dout must be 16-byte aligned with strides that are multiples of 4");
  WA_CHECK_ARG(wa_aligned16(a->x) && a->x_sb % xv == 0 && a->x_st % xv == 0 && a->x_sh % xv == 0,
               "wa_compress_kv_bwd: x must be 16-byte aligned with strides that are multiples of 16 bytes");
  WA_CHECK_ARG(a->dx == nullptr || (wa_aligned16(a->dx) && a->dx_sb % 4 == 0 && a->dx_st % 4 == 0 && a->dx_sh % 4 == 0),
               "wa_compress_kv_bwd: dx must be 16-byte aligned with strides that are multiples of 4");
  WA_CHECK_ARG(a->L <= INT32_MAX && a->proj_rank * a->proj_len <= INT32_MAX, "wa_compress_kv_bwd: sizes too large");
  const int64_t r_full = std::min(a->proj_rank, (n_first + a->block_size - 1) / a->block_size);
  const int64_t n_seg = (a->L + a->segment_len - 1) / a->segment_len;
  CompressBwdParams cp{a->dout, a->d_sb, a->d_st, a->d_sh, a->x, a->x_sb, a->x_st, a->x_sh, a->x_dtype,
                       a->proj, a->proj_dtype, (int)a->proj_rank, (int)a->proj_len,
                       (int)a->B, (int)a->L, (int)a->H, (int)a->D, (int)a->segment_len, (int)a->block_size,
                       (int)n_first, (int)r_full, (int)n_seg,
                       a->dx, a->dx_sb, a->dx_st, a->dx_sh, a->dx_accumulate,
                       a->dproj, a->dproj_accumulate, (float*)a->workspace};
  hipStream_t s = (hipStream_t)stream;
  if (a->B > 0 && a->dx) {
    const int64_t tps = (n_first + kDxTokens - 1) / kDxTokens;
    const int64_t cols = a->H * a->D / 4;
    dim3 grid((unsigned)(n_seg * tps), (unsigned)((cols + kDxThreads - 1) / kDxThreads), (unsigned)a->B);
    hipLaunchKernelGGL(compress_bwd_dx_kernel, grid, dim3(kDxThreads), 0, s, cp);
    const int rc = wa_launch_status("compress_kv_bwd (dx)");
    if (rc != WA_OK) return rc;
  }
  if (a->dproj) {
    if (a->B > 0) {
      dim3 grid((unsigned)((n_first + 63) / 64), (unsigned)n_seg);
      if (r_full <= 16) hipLaunchKernelGGL(compress_bwd_dproj_kernel<16>, grid, dim3(256), 0, s, cp);
      else if (r_full <= 32) hipLaunchKernelGGL(compress_bwd_dproj_kernel<32>, grid, dim3(256), 0, s, cp);
      else if (r_full <= 64) hipLaunchKernelGGL(compress_bwd_dproj_kernel<64>, grid, dim3(256), 0, s, cp);
      else hipLaunchKernelGGL(compress_bwd_dproj_kernel<128>, grid, dim3(256), 0, s, cp);
      const int rc = wa_launch_status("compress_kv_bwd (dproj)");
      if (rc != WA_OK) return rc;
    } else {
      cp.n_seg = 0;  // no batches: every partial is zero
    }
    const int64_t total = a->proj_rank * a->proj_len;
    hipLaunchKernelGGL(compress_bwd_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, cp);
    return wa_launch_status("compress_kv_bwd (reduce)");
  }
  return WA_OK;
}

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
  // bf16 x with 16-byte aligned rows (and a rank of at most 32): the streaming kernel
  const int64_t slab = ((a->L - 1) * a->x_st + a->D) * 2;
  const int64_t rank_used = std::min<int64_t>(a->proj_rank, (std::min<int64_t>(a->segment_len, a->L) + a->block_size - 1) /
                                                                a->block_size);
  if ((a->D == 128 || a->D == 64) && a->x_dtype == WA_BF16 && wa_aligned16(a->x) && a->x_sb % 8 == 0 &&
      a->x_st % 8 == 0 && a->x_sh % 8 == 0 && slab < ((int64_t)1 << 31) && rank_used <= 32 &&
      a->proj_dtype == WA_BF16 && (((uintptr_t)a->proj) & 3) == 0 && a->proj_len % 2 == 0 &&
      a->proj_rank * a->proj_len * 2 < ((int64_t)1 << 31)) {
    cp.x_slab = slab;
    if (a->D == 128) hipLaunchKernelGGL(compress_stream_kernel<128>, grid, dim3(256), 0, s, cp);
    else hipLaunchKernelGGL(compress_stream_kernel<64>, grid, dim3(128), 0, s, cp);
    return wa_launch_status("compress_kv");
  }
  if (a->D == 128) hipLaunchKernelGGL(compress_kernel<128>, grid, dim3(256), 0, s, cp);
  else if (a->D == 64) hipLaunchKernelGGL(compress_kernel<64>, grid, dim3(256), 0, s, cp);
  else hipLaunchKernelGGL(compress_kernel<32>, grid, dim3(256), 0, s, cp);
  return wa_launch_status("compress_kv");
}
