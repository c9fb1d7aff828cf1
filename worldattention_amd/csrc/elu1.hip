// Kernelized linear attention with phi(x) = elu(x) + 1 (the north-star "linear-global" heads):
//   state:   S^T[d, e] = sum_t v[t, d] phi(k[t, e]),   z[e] = sum_t phi(k[t, e])
//   readout: o[q, d] = sum_e phi(q[q, e]) S^T[d, e] / (phi(q) . z)   (+ gated-fusion epilogue)
// There is no reference counterpart: the reference's linear branch is the low-rank softmax branch
// (wan/modules/hsa/attention.py:64-118), kept in linear.hip.
//
// gfx950 layout. Both products contract over a dimension that is contiguous in memory for one of
// the operands only, so the state kernel stages row-major [token][channel] tiles in LDS and feeds
// BOTH MFMA operands with transpose reads (ds_read_b64_tr_b16), while the next 64-token tile
// streams into registers. The readout stages S^T once per workgroup in LDS as a bf16 hi + lo pair
// (two MFMAs keep ~16 mantissa bits of the fp32 state).
#include <algorithm>

#include "tile.h"

namespace {

typedef wa_s16x4 s16x4;
#define WA_LDS4(p) WA_LDS_S16X4(p)

// Row swizzles of 16-byte chunks (see bsa_fwd.hip): transpose reads cover 4 rows x 32 bytes per
// 16 lanes; 128-bit reads cover 16 rows x 16 bytes.
__device__ __forceinline__ int tr_swizzle(int r) { return 2 * (r & 3); }
template <int D>
__device__ __forceinline__ int row_swizzle(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }

// MFMA operand fragment of a row-major, tr-swizzled [rows][D] bf16 LDS tile for a contraction over
// rows [16c, 16c + 16): lane (l32, g) receives rows 16c + 8g + e (e = 0..7) at column col0 + l32.
// Transpose-read semantics (per 16-lane group): result lane i, element r comes from element i % 4
// of source lane 4r + i / 4.
template <int D>
__device__ __forceinline__ bf16x8 tr_frag(const bf16_t* buf, int c, int col0, int lane) {
  const int G = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
  bf16x8 a;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int row = 16 * c + 8 * (G >> 1) + 4 * hf + r;
    const int col = col0 + 16 * (G & 1) + 4 * q;
    const int slot = (col >> 3) ^ tr_swizzle(row);
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(WA_LDS4(buf + row * D + slot * 8 + (col & 7)));
    const bf16x4 b = __builtin_bit_cast(bf16x4, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[4 * hf + e] = b[e];
  }
  return a;
}

template <typename T>
__device__ __forceinline__ void load_row8(const T* src, float (&f)[8]);
template <>
__device__ __forceinline__ void load_row8<bf16_t>(const bf16_t* src, float (&f)[8]) {
  const bf16x8 v = *(const bf16x8*)src;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
}
template <>
__device__ __forceinline__ void load_row8<float>(const float* src, float (&f)[8]) {
  const f32x4 a = *(const f32x4*)src, b = *(const f32x4*)(src + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[e + 4] = b[e];
  }
}

// =============================================================================================
// state: one workgroup per (token chunk, head slot, batch) writes a partial S^T and z; a second
// pass sums the chunk partials in a fixed order (bitwise reproducible).
// =============================================================================================
struct StateParams {
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  int H, L, n_heads, n_chunks, chunk_len, B;
  const int32_t* heads;
  float* part;  // [n_chunks][B][n_heads][D*D + D]
  float* state; float* zsum;
};

template <int D, typename T>
__global__ void __launch_bounds__(256) elu1_state_kernel(StateParams p) {
  constexpr int TC = 64;                 // tokens per LDS tile
  constexpr int CPR = D / 8;             // 8-element chunks per row
  constexpr int UPT = TC * CPR / 256;    // chunks per thread per tensor (4 or 2)
  constexpr int NT = D / 32;             // 32-wide tiles along d and e
  constexpr int TPW = NT * NT / 4;       // output tiles per wave (4 or 1)
  __shared__ __attribute__((aligned(1024))) bf16_t kb[2][TC * D];
  __shared__ __attribute__((aligned(1024))) bf16_t vb[2][TC * D];

  const int chunk = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int tbeg = chunk * p.chunk_len;
  const int tend = min(p.L, tbeg + p.chunk_len);
  const int c8 = tid % CPR, row0 = tid / CPR;  // this thread's chunk column and first row
  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + c8 * 8;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + c8 * 8;

  // wave w owns output tiles (dt, et): D = 128 -> dt = w, et = 0..3; D = 64 -> (w / 2, w % 2)
  f32x16 acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = f32x16{};
  float zacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) zacc[e] = 0.f;

  // one register stage of the next 64-token tile (raw values); an LDS double buffer holds bf16
  // phi(k) / v of the tile being multiplied
  float kr[1][UPT][8], vr[1][UPT][8];
#define WA_ELU1_LOAD(S, T0)                                                         \
  _Pragma("unroll") for (int i = 0; i < UPT; ++i) {                                 \
    const int t = (T0) + row0 + i * (256 / CPR);                                    \
    if (t < tend) {                                                                 \
      load_row8<T>(kbase + (int64_t)t * p.k_st, kr[S][i]);                          \
      load_row8<T>(vbase + (int64_t)t * p.v_st, vr[S][i]);                          \
    } else {                                                                        \
      _Pragma("unroll") for (int e = 0; e < 8; ++e) kr[S][i][e] = vr[S][i][e] = 0.f; \
    }                                                                               \
  }
#define WA_ELU1_STORE(S, BUF, T0)                                           \
  _Pragma("unroll") for (int i = 0; i < UPT; ++i) {                         \
    const int r = row0 + i * (256 / CPR);                                   \
    const bool ok = (T0) + r < tend;                                        \
    bf16x8 kk, vv;                                                          \
    _Pragma("unroll") for (int e = 0; e < 8; ++e) {                         \
      const float ph = ok ? wa_bf16_round(elu1f(kr[S][i][e])) : 0.f;       \
      zacc[e] += ph;                                                        \
      kk[e] = (bf16_t)ph;                                                   \
      vv[e] = (bf16_t)vr[S][i][e];                                          \
    }                                                                       \
    const int slot = c8 ^ tr_swizzle(r);                                    \
    *(bf16x8*)(&kb[BUF][r * D + slot * 8]) = kk;                            \
    *(bf16x8*)(&vb[BUF][r * D + slot * 8]) = vv;                            \
  }
#define WA_ELU1_MMA(BUF)                                                    \
  _Pragma("unroll") for (int c = 0; c < TC / 16; ++c) {                     \
    _Pragma("unroll") for (int i = 0; i < TPW; ++i) {                       \
      const int dt = D == 128 ? w : (w >> 1);                               \
      const int et = D == 128 ? i : (w & 1);                                \
      const bf16x8 a = tr_frag<D>(vb[BUF], c, 32 * dt, lane);               \
      const bf16x8 bb = tr_frag<D>(kb[BUF], c, 32 * et, lane);              \
      acc[i] = wa_mfma32(a, bb, acc[i]);                                    \
    }                                                                       \
  }

  // tile t0 + TC streams into registers while tile t0 is multiplied (LDS buffers alternate;
  // unrolled by two so every index is static)
  int t0 = tbeg;
  if (t0 < tend) { WA_ELU1_LOAD(0, t0) }
  while (t0 < tend) {
    WA_ELU1_STORE(0, 0, t0)
    if (t0 + TC < tend) { WA_ELU1_LOAD(0, t0 + TC) }
    __syncthreads();  // LDS buffer 0 complete; every wave is past the tile before it
    WA_ELU1_MMA(0)
    t0 += TC;
    if (t0 >= tend) break;
    WA_ELU1_STORE(0, 1, t0)
    if (t0 + TC < tend) { WA_ELU1_LOAD(0, t0 + TC) }
    __syncthreads();
    WA_ELU1_MMA(1)
    t0 += TC;
  }
#undef WA_ELU1_STORE
#undef WA_ELU1_MMA
#undef WA_ELU1_LOAD

  float* part = p.part + (((int64_t)chunk * p.B + b) * p.n_heads + hs) * (int64_t)(D * D + D);
  // accumulator lane (e = 32 et + l32, g) holds d = 32 dt + 8 (r / 4) + 4 g + r % 4
  const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int dt = D == 128 ? w : (w >> 1);
    const int et = D == 128 ? i : (w & 1);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * dt + 8 * (r >> 2) + 4 * g + (r & 3);
      part[d * D + 32 * et + l32] = acc[i][r];
    }
  }
  // z: threads with the same chunk column c8 hold disjoint rows; reduce them in a fixed order
  __syncthreads();
  float* zbuf = (float*)kb;  // reuse the tile buffers: [256 threads][8]
#pragma unroll
  for (int e = 0; e < 8; ++e) zbuf[tid * 8 + e] = zacc[e];
  __syncthreads();
  if (tid < D) {
    const int cc = tid / 8, e = tid % 8;
    float s = 0.f;
    for (int r = 0; r < 256 / CPR; ++r) s += zbuf[(r * CPR + cc) * 8 + e];
    part[D * D + tid] = s;
  }
}

// bf16 K / V: raw [64 token][D] tiles stream global -> LDS by direct-to-LDS loads into a 4-stage
// ring. The loads are inline assembly that the compiler does not track: through the builtin it
// made the first LDS read of every tile wait for all loads in flight (s_waitcnt vmcnt(0)), which
// drained the ring each step; the waits below count the loads instead. The loop is software
// pipelined over tiles: while the MFMAs of tile `it` read its stage, the same waves apply phi in
// place to the K rows of tile it + 1, and tiles it + 2 and it + 3 stream in. One barrier per tile:
// it publishes the phi writes of tile it + 1 and frees the stage that tile it + 4 streams into.
// Most of the loop's VALU instructions are phi's (~8 per element), so z is summed on the MFMA pipe
// as a product with a ones row rather than by the phi pass. Rows past the chunk read
// zeros and get phi = 0 (as -inf), so they add nothing to S or z.
// Output tiles (dt, et) of S^T (NT x NT tiles of 32 x 32): wave w owns the TPW tiles of column et
// = w % NT in rows (w / NT) TPW + i, so its products share one phi(K) fragment per 16 tokens.
template <int NT, int TPW>
__device__ __forceinline__ int tile_d(int w, int i) { return (w / NT) * TPW + i; }
template <int NT, int TPW>
__device__ __forceinline__ int tile_e(int w, int) { return w % NT; }

template <int D, int NW>
__global__ void __launch_bounds__(64 * NW) elu1_state_dma_kernel(StateParams p) {
  constexpr int TC = 64, STAGES = 4, NTH = 64 * NW;
  constexpr int CPR = D / 8;              // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;           // rows per wave DMA instruction
  constexpr int NI = TC / (RPI * NW);     // DMA instructions per wave per tensor per tile
  constexpr int UPT = TC * CPR / NTH;     // chunks per thread in the phi pass
  constexpr int NT = D / 32, TPW = NT * NT / NW;
  static_assert(NI >= 1 && UPT >= 1 && TPW >= 1 && NT * NT == TPW * NW && NW % NT == 0, "bad wave count");
  __shared__ __attribute__((aligned(1024))) bf16_t kb[STAGES][TC * D];
  __shared__ __attribute__((aligned(1024))) bf16_t vb[STAGES][TC * D];

  const int chunk = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tbeg = chunk * p.chunk_len;
  const int tend = min(p.L, tbeg + p.chunk_len);
  const int ntiles = tend > tbeg ? (tend - tbeg + TC - 1) / TC : 0;
  const bf16_t* kbase = (const bf16_t*)p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16_t* vbase = (const bf16_t*)p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;

  // Tile loads through one buffer descriptor per tile and tensor (scalar work only), starting at
  // the tile's first row and ending at the chunk's last row, so rows past the chunk read zeros;
  // this lane's byte offsets within a tile are loop-invariant.
  int k_off[NI], v_off[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (i * NW + w) * RPI + lane / CPR, cc = (lane % CPR) ^ tr_swizzle(row);
    k_off[i] = (int)(row * p.k_st + cc * 8) * 2;
    v_off[i] = (int)(row * p.v_st + cc * 8) * 2;
  }
  auto issue = [&](int it) {
    const int t0 = tbeg + it * TC, st = it % STAGES, rows = min(TC, tend - t0);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kbase + (int64_t)t0 * p.k_st), (short)0, (int)((rows - 1) * p.k_st + D) * 2, WA_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vbase + (int64_t)t0 * p.v_st), (short)0, (int)((rows - 1) * p.v_st + D) * 2, WA_BUF_DWORD3);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r0 = (i * NW + w) * RPI;
      lds_dma16(krs, &kb[st][r0 * D], k_off[i]);
      lds_dma16(vrs, &vb[st][r0 * D], v_off[i]);
    }
  };

  f32x16 acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = f32x16{};
  // z = ones^T phi(K) on the MFMA pipe: every row of zt holds z over the wave's column tile (the
  // NW / NT waves of a column tile each sum all of it: no branch between the products; the first
  // one's is kept).
  f32x16 zt = f32x16{};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  const int c8 = tid % CPR;  // this thread's channel chunk in the phi pass

  // phi in place on the K rows of tile `it` (zero past the chunk)
  auto phi = [&](int it) {
    const int t0 = tbeg + it * TC;
    bf16_t* kt = kb[it % STAGES];
    bf16x8 x[UPT];
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int r = tid / CPR + u * (NTH / CPR);
      x[u] = *(const bf16x8*)(kt + r * D + ((c8 ^ tr_swizzle(r)) * 8));
    }
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int r = tid / CPR + u * (NTH / CPR);
      // a row past the chunk becomes -inf, whose phi is exp(-inf) = 0 (a bitwise blend: a
      // conditional phi, or a conditional assignment, compiled to branches)
      const unsigned past = 0u - (unsigned)(t0 + r >= tend);
      u32x4 xw = __builtin_bit_cast(u32x4, x[u]);
#pragma unroll
      for (int j = 0; j < 4; ++j) xw[j] = (xw[j] & ~past) | (0xff80ff80u & past);
      x[u] = __builtin_bit_cast(bf16x8, xw);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[u][e] = (bf16_t)elu1f((float)x[u][e]);
      *(bf16x8*)(kt + r * D + ((c8 ^ tr_swizzle(r)) * 8)) = x[u];
    }
  };
  // S^T tiles += V^T phi(K) over the 64 tokens of tile `it`
  auto products = [&](int it) {
    const int st = it % STAGES, et = tile_e<NT, TPW>(w, 0);
#pragma unroll
    for (int c = 0; c < TC / 16; ++c) {
      const bf16x8 bb = tr_frag<D>(kb[st], c, 32 * et, lane);
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const bf16x8 a = tr_frag<D>(vb[st], c, 32 * tile_d<NT, TPW>(w, i), lane);
        acc[i] = wa_mfma32(a, bb, acc[i]);
      }
      zt = wa_mfma32(ones, bb, zt);
    }
  };

  // Tiles 0 and 1 first, tile 2 once tile 0 has landed: with every workgroup of the launch
  // starting at once, a smaller first burst brings tile 0 in sooner.
  for (int it = 0; it < min(ntiles, 2); ++it) issue(it);
  if (ntiles > 0) {
    if (ntiles >= 2) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    if (ntiles > 2) issue(2);
    phi(0);
  }
  for (int it = 0; it < ntiles; ++it) {
    // Issued so far: tiles up to it + 2. Tile it + 1 must have landed (tile it + 2 may stream),
    // and every wave's phi writes of tile it and products of tile it - 1 be done.
    if (it + 2 < ntiles) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * NI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (it + STAGES - 1 < ntiles) issue(it + STAGES - 1);  // into the stage of tile it - 1
    products(it);
    // after the last tile every row is past the chunk: phi writes zeros into a stage nothing
    // reads again (unconditional, so one basic block holds both)
    phi(it + 1);
  }

  float* part = p.part + (((int64_t)chunk * p.B + b) * p.n_heads + hs) * (int64_t)(D * D + D);
  const int g = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int dt = tile_d<NT, TPW>(w, i), et = tile_e<NT, TPW>(w, i);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * dt + 8 * (r >> 2) + 4 * g + (r & 3);
      part[d * D + 32 * et + l32] = acc[i][r];
    }
  }
  // z over column tile w: row 0 of zt (lanes 0..31)
  if (w < NT && g == 0) part[D * D + 32 * w + l32] = zt[0];
}

// Sum of the chunk partials, four bytes-in-flight-heavy waves per 64 float4 positions: wave q sums
// the chunks of quarter q (up to 8 float4 loads in flight per lane), then wave 0 adds the four
// quarter sums, always in the same order (bitwise reproducible).
__global__ void __launch_bounds__(256) elu1_reduce_kernel(StateParams p, int D) {
  __shared__ f32x4 qsum[4][64];
  const int64_t per = (int64_t)D * D + D;  // a multiple of 4: no float4 straddles S^T and z
  const int64_t total = (int64_t)p.B * p.n_heads * per;
  const int64_t i4 = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  const int q = threadIdx.x >> 6;
  const int c0 = (int)((int64_t)p.n_chunks * q / 4), c1 = (int)((int64_t)p.n_chunks * (q + 1) / 4);
  f32x4 a = {0.f, 0.f, 0.f, 0.f};
  if (i4 * 4 < total) {
    const f32x4* src = (const f32x4*)p.part + i4;
    const int64_t stride = total / 4;
    int c = c0;
    for (; c + 8 <= c1; c += 8) {
      f32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)(c + j) * stride];
#pragma unroll
      for (int j = 0; j < 8; ++j) a += v[j];
    }
    for (; c < c1; ++c) a += src[(int64_t)c * stride];
  }
  qsum[q][threadIdx.x & 63] = a;
  __syncthreads();
  if (q != 0 || i4 * 4 >= total) return;
  const f32x4 s = (qsum[0][threadIdx.x] + qsum[1][threadIdx.x]) + (qsum[2][threadIdx.x] + qsum[3][threadIdx.x]);
  const int64_t bh = i4 * 4 / per, r = i4 * 4 % per;
  float* dst = r < (int64_t)D * D ? p.state + bh * D * D + r : p.zsum + bh * D + (r - (int64_t)D * D);
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[e] = s[e];
}

// =============================================================================================
// readout: one workgroup of 8 waves per (128-query tile, head slot, batch). Wave w owns 32
// queries (w % 4) and half of the output channels (w / 4): the two halves share the staged S^T and
// both compute phi(q) and the denominator of their queries, which halves each wave's MFMA and
// epilogue work and puts two waves on every SIMD.
// =============================================================================================
struct ReadoutParams {
  const void* q; int64_t q_sb, q_st, q_sh; int q_dtype;
  const float* state; const float* zsum;
  void* o; int64_t o_sb, o_st, o_sh; int o_dtype;
  int H, L, n_heads;
  const int32_t* heads;
  int epilogue;
  const bf16_t* gate_w; const float* gate_b;
  int gate_pre_bf16, gate_out_bf16, lin_round_bf16;
};

// HOT != 0 fixes the HSA forward's bf16 configuration at compile time: bf16 q and o, gated
// epilogue with gate weights, bf16 rounding of the linear output and of the gate, and of the gate
// pre-activation for HOT = 1 only (a bf16 gate layer) but not for HOT = 2 (an fp32 one). HOT = 0
// reads each option from the params.
template <int D, int HOT>
__global__ void __launch_bounds__(512) elu1_readout_kernel(ReadoutParams p) {
  constexpr int DC = D / 16, DT = D / 32, DTW = DT / 2, CPR = D / 8;
  __shared__ __attribute__((aligned(1024))) bf16_t s_hi[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t s_lo[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t s_w[D * D];
  __shared__ float s_z[D];
  __shared__ float s_gb[D];
  const int tile = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int qg = w & 3, dp = w >> 2;
  const float* S = p.state + ((int64_t)b * p.n_heads + hs) * D * D;
  const bool q_bf = HOT || p.q_dtype == WA_BF16;
  const bool o_bf = HOT || p.o_dtype == WA_BF16;
  const bool need_gate = HOT || p.epilogue == WA_EPI_GATED;
  const bool use_w = HOT ? true : (need_gate && p.gate_w);
  const bool pre_bf = HOT ? HOT == 1 : p.gate_pre_bf16;
  const bool gout_bf = HOT || p.gate_out_bf16;
  const bool lin_bf = HOT || p.lin_round_bf16;

  // Every global read of the workgroup is issued up front so the latencies overlap: this lane's
  // query row, S^T (staged as bf16 hi + lo), the gate weights, z and the gate bias (both to LDS).
  const int qi = tile * 128 + qg * 32 + l32;
  const bool q_ok = qi < p.L;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)(q_ok ? qi : 0) * p.q_st + (int64_t)h * p.q_sh;
  float qraw[DC][8];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    if (q_bf) load_row8<bf16_t>((const bf16_t*)p.q + qoff + c * 16 + g * 8, qraw[c]);
    else load_row8<float>((const float*)p.q + qoff + c * 16 + g * 8, qraw[c]);
  }
  constexpr int SU = D * CPR / 512;  // 8-element units per thread (4 or 1)
  f32x4 x0[SU], x1[SU];
  bf16x8 wv[SU];
#pragma unroll
  for (int k = 0; k < SU; ++k) {
    const int u = tid + 512 * k, d = u / CPR, cc = u % CPR;
    x0[k] = *(const f32x4*)(S + d * D + cc * 8);
    x1[k] = *(const f32x4*)(S + d * D + cc * 8 + 4);
    if (use_w) wv[k] = *(const bf16x8*)(p.gate_w + d * D + cc * 8);
  }
  for (int e = tid; e < D; e += 512) {
    s_z[e] = p.zsum[((int64_t)b * p.n_heads + hs) * D + e];
    s_gb[e] = p.gate_b ? p.gate_b[e] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < SU; ++k) {
    const int u = tid + 512 * k, d = u / CPR, cc = u % CPR;
    bf16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hi[e] = (bf16_t)x0[k][e];
      lo[e] = (bf16_t)(x0[k][e] - (float)hi[e]);
      hi[e + 4] = (bf16_t)x1[k][e];
      lo[e + 4] = (bf16_t)(x1[k][e] - (float)hi[e + 4]);
    }
    const int slot = cc ^ row_swizzle<D>(d);
    *(bf16x8*)(s_hi + d * D + slot * 8) = hi;
    *(bf16x8*)(s_lo + d * D + slot * 8) = lo;
    if (use_w) *(bf16x8*)(s_w + d * D + slot * 8) = wv[k];
  }
  bf16x8 qf[DC], phf[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    float* f = qraw[c];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (!q_ok) f[e] = 0.f;
      qf[c][e] = (bf16_t)f[e];
      phf[c][e] = (bf16_t)elu1f(f[e]);
    }
  }
  __syncthreads();
  float den = 0.f;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) den = fmaf((float)phf[c][e], s_z[c * 16 + g * 8 + e], den);
  }
  den += __shfl_xor(den, 32, 64);

  // O^T[d, q] = S^T[d, :] phi(Q)^T[:, q] over this wave's channel tiles; A fragment: row
  // d = 32 T + l32, chunk 2c + g
  f32x16 oacc[DTW], gacc[DTW];
  const int rs = row_swizzle<D>(l32);
#pragma unroll
  for (int t = 0; t < DTW; ++t) {
    const int T = dp * DTW + t;
    oacc[t] = f32x16{};
    gacc[t] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const int off = (32 * T + l32) * D + ((2 * c + g) ^ rs) * 8;
      oacc[t] = wa_mfma32(*(const bf16x8*)(s_hi + off), phf[c], oacc[t]);
      oacc[t] = wa_mfma32(*(const bf16x8*)(s_lo + off), phf[c], oacc[t]);
      if (use_w) gacc[t] = wa_mfma32(*(const bf16x8*)(s_w + off), qf[c], gacc[t]);
    }
  }
  if (!q_ok) return;
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
  for (int t = 0; t < DTW; ++t) {
    const int T = dp * DTW + t;
    // every global read of the tile (gate bias or q) before its stores (see bsa_fwd.hip)
    float pre[4][4];
    if (need_gate) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = T * 32 + 8 * rq + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pre[rq][i] = use_w ? gacc[t][rq * 4 + i] + s_gb[d0 + i] : wa_load_f(p.q, qoff + d0 + i, p.q_dtype);
      }
    }
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = T * 32 + 8 * rq + 4 * g;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = oacc[t][rq * 4 + i] * inv;
        if (lin_bf) a = wa_bf16_round(a);
        if (need_gate) {
          float pr = pre[rq][i];
          if (pre_bf) pr = wa_bf16_round(pr);
          float gs = wa_sigmoid(pr);
          if (gout_bf) gs = wa_bf16_round(gs);
          a = wa_mul_rn(a, gs);
        }
        val[i] = a;
      }
      if (o_bf) {
        bf16x4 ov = {(bf16_t)val[0], (bf16_t)val[1], (bf16_t)val[2], (bf16_t)val[3]};
        *(bf16x4*)((bf16_t*)p.o + oo + d0) = ov;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) ((float*)p.o)[oo + d0 + i] = val[i];
      }
    }
  }
}

// =============================================================================================
// backward. With n = phi(q) S, den = phi(q) . z, o = n / den and g = dL/do (per head, batch):
//   dn = g / den,  dden = -(g . o) / den,  dphi(q) = S^T-contraction of dn + dden z,
//   dS^T[d, e] = sum_q dn[q, d] phi(q)[q, e],  dz = sum_q dden[q] phi(q)[q, :],
//   dphi(k)[t, e] = sum_d v[t, d] dS^T[d, e] + dz[e],  dv[t, d] = sum_e dS^T[d, e] phi(k)[t, e],
//   and dx = dphi(x) * phi'(x) with phi'(x) = 1 (x > 0) or e^x.
// =============================================================================================
struct Elu1BwdParams {
  const void* q; int64_t q_sb, q_st, q_sh; int q_dtype;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh; int kv_dtype;
  const void* g; int64_t g_sb, g_st, g_sh; int g_dtype;
  const float* state; const float* zsum;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int dq_acc;
  void* dk; int64_t dk_sb, dk_st, dk_sh; int dk_acc;
  void* dv; int64_t dv_sb, dv_st, dv_sh; int dv_acc;
  int dkv_bf16;  // dk / dv are bf16 (written once) instead of fp32
  int kv_groups_per_wg;  // 32-token groups per workgroup of the bf16 key-side kernel
  const int32_t* heads; int n_heads, H, B, Lq, Lkv, n_qt;
  float* part;    // [n_qt][B][n_heads][D*D + D]
  float* dstate;  // [B][n_heads][D*D]
  float* dz;      // [B][n_heads][D]
};

__device__ __forceinline__ float elu1_grad(float x) { return x > 0.f ? 1.f : __expf(x); }

__device__ __forceinline__ void load4_any(const void* base, int64_t i, int dtype, float (&f)[4]) {
  if (dtype == WA_BF16) {
    const bf16x4 v = *(const bf16x4*)((const bf16_t*)base + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = (float)v[e];
  } else {
    const f32x4 v = *(const f32x4*)((const float*)base + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = v[e];
  }
}

__device__ __forceinline__ void load8_any(const void* base, int64_t i, int dtype, float (&f)[8]) {
  if (dtype == WA_BF16) load_row8<bf16_t>((const bf16_t*)base + i, f);
  else load_row8<float>((const float*)base + i, f);
}

// Stages an fp32 [D][D] matrix as bf16 hi + lo dual-swizzled tiles (rows = first index).
template <int D, int NT = 256>
__device__ __forceinline__ void stage_hilo(const float* S, bf16_t* hi_t, bf16_t* lo_t, int tid) {
  constexpr int CPR = D / 8, SU = D * CPR / NT;
  f32x4 x0[SU], x1[SU];
#pragma unroll
  for (int k = 0; k < SU; ++k) {
    const int u = tid + NT * k, d = u / CPR, cc = u % CPR;
    x0[k] = *(const f32x4*)(S + d * D + cc * 8);
    x1[k] = *(const f32x4*)(S + d * D + cc * 8 + 4);
  }
#pragma unroll
  for (int k = 0; k < SU; ++k) {
    const int u = tid + NT * k, d = u / CPR, cc = u % CPR;
    bf16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      hi[e] = (bf16_t)x0[k][e];
      lo[e] = (bf16_t)(x0[k][e] - (float)hi[e]);
      hi[e + 4] = (bf16_t)x1[k][e];
      lo[e + 4] = (bf16_t)(x1[k][e] - (float)hi[e + 4]);
    }
    tile_put8<D>(hi_t, d, cc, hi);
    tile_put8<D>(lo_t, d, cc, lo);
  }
}

// Query side: one workgroup of 8 waves per (128-query tile, head slot, batch), two waves per
// SIMD. Wave w owns queries 32 (w & 3).. and the channel half w >> 2 of each product's output; both
// halves form phi(q) and the denominator of their queries (the contraction runs over all channels).
template <int D>
__global__ void __launch_bounds__(512) elu1_bwd_q_kernel(Elu1BwdParams p) {
  constexpr int DC = D / 16, DT = D / 32, TTW = DT / 2;
  __shared__ __attribute__((aligned(1024))) bf16_t s_hi[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t s_lo[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t t_dn[128 * D];
  __shared__ __attribute__((aligned(1024))) bf16_t t_ph[128 * D];
  __shared__ float s_z[D], s_dd[128], s_go[2][128], s_dz[4][D];
  const int tile = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int half = w >> 2;
  const int64_t bh = (int64_t)b * p.n_heads + hs;
  stage_hilo<D, 512>(p.state + bh * D * D, s_hi, s_lo, tid);
  for (int e = tid; e < D; e += 512) s_z[e] = p.zsum[bh * D + e];
  __syncthreads();

  const int ql = (w & 3) * 32 + l32, qi = tile * 128 + ql;
  const bool q_ok = qi < p.Lq;
  const int64_t qoff = (int64_t)b * p.q_sb + (int64_t)(q_ok ? qi : 0) * p.q_st + (int64_t)h * p.q_sh;
  const int64_t goff = (int64_t)b * p.g_sb + (int64_t)(q_ok ? qi : 0) * p.g_st + (int64_t)h * p.g_sh;
  bf16x8 phf[DC];
  float den = 0.f;
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    float f[8];
    load8_any(p.q, qoff + c * 16 + g * 8, p.q_dtype, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ph = q_ok ? wa_bf16_round(elu1f(f[e])) : 0.f;
      phf[c][e] = (bf16_t)ph;
      den = fmaf(ph, s_z[c * 16 + g * 8 + e], den);
    }
    if (c / (DC / 2) == half) tile_put8<D>(t_ph, ql, 2 * c + g, phf[c]);
  }
  den += __shfl_xor(den, 32, 64);
  const float inv = q_ok && den > 0.f ? 1.f / den : 0.f;

  // n^T = S^T phi(q)^T for this half's output tiles, then o, (g . o), dn (accumulator layout:
  // lane q, d = 32t + 8(r/4) + 4g + r%4)
  f32x16 acc[TTW];
#pragma unroll
  for (int k = 0; k < TTW; ++k) {
    const int t = half * TTW + k;
    acc[k] = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      acc[k] = wa_mfma32(tile_row8<D>(s_hi, 32 * t + l32, 2 * c + g), phf[c], acc[k]);
      acc[k] = wa_mfma32(tile_row8<D>(s_lo, 32 * t + l32, 2 * c + g), phf[c], acc[k]);
    }
  }
  float go = 0.f;
#pragma unroll
  for (int k = 0; k < TTW; ++k) {
    const int t = half * TTW + k;
    float gv[4][4];
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) load4_any(p.g, goff + 32 * t + 8 * rq + 4 * g, p.g_dtype, gv[rq]);
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      bf16x4 dn4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gg = q_ok ? gv[rq][i] : 0.f;
        go = fmaf(gg, acc[k][rq * 4 + i] * inv, go);
        dn4[i] = (bf16_t)(gg * inv);
      }
      // t_dn[q][d]: 4 consecutive channels of one 16-byte chunk
      const int d0 = 32 * t + 8 * rq + 4 * g;
      *(bf16x4*)(t_dn + ql * D + (((d0 >> 3) ^ dual_swizzle<D>(ql)) * 8) + (d0 & 7)) = dn4;
    }
  }
  go += __shfl_xor(go, 32, 64);
  if (g == 0) s_go[half][ql] = go;
  __syncthreads();  // t_dn, t_ph and both halves of (g . o) complete
  const float dden = -(s_go[0][ql] + s_go[1][ql]) * inv;
  if (g == 0 && half == 0) s_dd[ql] = q_ok ? dden : 0.f;

  // dphi(q)^T[e, q] = sum_d S^T[d, e] dn[q, d] (+ dden z[e]) for this half's channels e
#pragma unroll
  for (int k = 0; k < TTW; ++k) {
    const int et = half * TTW + k;
    f32x16 da = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const bf16x8 dn8 = tile_row8<D>(t_dn, ql, 2 * c + g);
      da = wa_mfma32(tile_tr8n<D>(s_hi, c, 32 * et, lane), dn8, da);
      da = wa_mfma32(tile_tr8n<D>(s_lo, c, 32 * et, lane), dn8, da);
    }
    if (q_ok) {
      // all reads (q and, when accumulating, the previous dq) before any store
      float* dst = p.dq + (int64_t)b * p.dq_sb + (int64_t)qi * p.dq_st + (int64_t)h * p.dq_sh;
      float qv[4][4], prev[4][4];
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int e0 = 32 * et + 8 * rq + 4 * g;
        load4_any(p.q, qoff + e0, p.q_dtype, qv[rq]);
#pragma unroll
        for (int i = 0; i < 4; ++i) prev[rq][i] = p.dq_acc ? dst[e0 + i] : 0.f;
      }
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int e0 = 32 * et + 8 * rq + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dst[e0 + i] = prev[rq][i] + (da[rq * 4 + i] + dden * s_z[e0 + i]) * elu1_grad(qv[rq][i]);
      }
    }
  }
  __syncthreads();  // s_dd complete

  // partial dS^T[d, e] = sum_q dn[q, d] phi(q)[q, e] over this tile (both operands transposed):
  // DT x DT output tiles spread over the 8 waves
  float* part = p.part + (((int64_t)tile * p.B + b) * p.n_heads + hs) * (int64_t)(D * D + D);
  for (int i = w; i < DT * DT; i += 8) {
    const int dt = i / DT, et = i % DT;
    f32x16 pa = f32x16{};
#pragma unroll
    for (int c = 0; c < 8; ++c) pa = wa_mfma32(tile_tr8<D>(t_dn, c, 32 * dt, lane), tile_tr8<D>(t_ph, c, 32 * et, lane), pa);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * dt + 8 * (r >> 2) + 4 * g + (r & 3);
      part[d * D + 32 * et + l32] = pa[r];
    }
  }
  // dz partial: per channel e four 32-query chains in fixed order, added in order
  if (tid < 4 * D) {
    const int e = tid % D, q4 = tid / D;
    float sz = 0.f;
    for (int k = 0; k < 32; ++k) {
      const int qq = q4 * 32 + k;
      sz = fmaf(s_dd[qq], (float)t_ph[qq * D + (((e >> 3) ^ dual_swizzle<D>(qq)) * 8) + (e & 7)], sz);
    }
    s_dz[q4][e] = sz;
  }
  __syncthreads();
  if (tid < D) part[D * D + tid] = ((s_dz[0][tid] + s_dz[1][tid]) + s_dz[2][tid]) + s_dz[3][tid];
}

// Key side: one workgroup per (128-token tile, head slot, batch), wave w = tokens 32w..
template <int D>
__global__ void __launch_bounds__(256) elu1_bwd_kv_kernel(Elu1BwdParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(1024))) bf16_t s_hi[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t s_lo[D * D];
  __shared__ float s_z[D];
  const int tile = blockIdx.x, hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int64_t bh = (int64_t)b * p.n_heads + hs;
  stage_hilo<D>(p.dstate + bh * D * D, s_hi, s_lo, tid);
  for (int e = tid; e < D; e += 256) s_z[e] = p.dz[bh * D + e];
  __syncthreads();

  const int tl = tile * 128 + w * 32 + l32;  // this lane's token as an A-operand row
  const bool t_ok = tl < p.Lkv;
  const int64_t koff = (int64_t)b * p.k_sb + (int64_t)(t_ok ? tl : 0) * p.k_st + (int64_t)h * p.k_sh;
  const int64_t voff = (int64_t)b * p.v_sb + (int64_t)(t_ok ? tl : 0) * p.v_st + (int64_t)h * p.v_sh;
  bf16x8 vf[DC], pk[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    float fk[8], fv[8];
    load8_any(p.k, koff + c * 16 + g * 8, p.kv_dtype, fk);
    load8_any(p.v, voff + c * 16 + g * 8, p.kv_dtype, fv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pk[c][e] = (bf16_t)(t_ok ? elu1f(fk[e]) : 0.f);
      vf[c][e] = (bf16_t)(t_ok ? fv[e] : 0.f);
    }
  }
  const int tb = tile * 128 + w * 32;  // accumulator rows: tokens tb + 8(r/4) + 4g + r%4
  // one 32-channel column tile at a time (unrolled, the tiles' epilogues spill registers)
#pragma unroll 1
  for (int jt = 0; jt < DT; ++jt) {
    f32x16 dk = f32x16{}, dv = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      // dphi(k)[t, e] = sum_d v[t, d] dS^T[d, e]   (B: column e of dS^T, rows d natural order)
      dk = wa_mfma32(vf[c], tile_tr8n<D>(s_hi, c, 32 * jt, lane), dk);
      dk = wa_mfma32(vf[c], tile_tr8n<D>(s_lo, c, 32 * jt, lane), dk);
      // dv[t, d] = sum_e phi(k)[t, e] dS^T[d, e]   (B: row d of dS^T)
      dv = wa_mfma32(pk[c], tile_row8<D>(s_hi, 32 * jt + l32, 2 * c + g), dv);
      dv = wa_mfma32(pk[c], tile_row8<D>(s_lo, 32 * jt + l32, 2 * c + g), dv);
    }
    const int col = 32 * jt + l32;
    // all reads (k and, when accumulating, the previous dk / dv) before any store
    float kx[16], prk[16], prv[16];
    const int64_t dk0 = (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh + col;
    const int64_t dv0 = (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh + col;
    float* dk_col = (float*)p.dk + dk0;
    float* dv_col = (float*)p.dv + dv0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = tb + 8 * (r >> 2) + 4 * g + (r & 3);
      const bool in = t < p.Lkv;
      const int64_t ko = (int64_t)b * p.k_sb + (int64_t)(in ? t : 0) * p.k_st + (int64_t)h * p.k_sh + col;
      kx[r] = p.kv_dtype == WA_BF16 ? (float)((const bf16_t*)p.k)[ko] : ((const float*)p.k)[ko];
      prk[r] = p.dk_acc && in ? dk_col[(int64_t)t * p.dk_st] : 0.f;
      prv[r] = p.dv_acc && in ? dv_col[(int64_t)t * p.dv_st] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = tb + 8 * (r >> 2) + 4 * g + (r & 3);
      if (t < p.Lkv) {
        const float gk = prk[r] + (dk[r] + s_z[col]) * elu1_grad(kx[r]), gv = prv[r] + dv[r];
        if (p.dkv_bf16) {
          ((bf16_t*)p.dk)[dk0 + (int64_t)t * p.dk_st] = (bf16_t)gk;
          ((bf16_t*)p.dv)[dv0 + (int64_t)t * p.dv_st] = (bf16_t)gv;
        } else {
          dk_col[(int64_t)t * p.dk_st] = gk;
          dv_col[(int64_t)t * p.dv_st] = gv;
        }
      }
    }
  }
}

// Key side, bf16 K / V in and bf16 dK / dV out (written once): the same products as
// elu1_bwd_kv_kernel, transposed so that a lane owns a token (accumulator layout: lane = token,
// registers = channels): dK^T[e, t] = sum_d dS^T[d, e] v[t, d], dV^T[d, t] = sum_e dS^T[d, e]
// phi(k)[t, e]. A workgroup stages the state gradient once (bf16 hi + lo: 64 KB at D = 128, two
// workgroups per CU) and its waves then walk 32-token groups of the workgroup's token run on their
// own, without barriers: K and V rows load straight into MFMA fragments, the next group's loads
// go out once the last column tile's products have read the fragments (before that tile's stores:
// on gfx9 loads and stores share one counter, so a load issued after a store waits for it), and
// each lane writes 8 channels (16 bytes) of its token per store, the two lanes of a token having
// swapped halves (with 8-byte stores the stores cost ~20 us of a ~46 us launch at cfg 5). The dK factor elu1'(k) comes from the K
// fragments: the two lanes of a token exchange the halves of their 16-byte chunks. (Holding the
// next group's fragments in registers for the whole group needs ~320 registers: one wave per
// SIMD, slower.)
// value of lane ^ 32 (g = lane >> 5): the gfx950 half-wave swap
__device__ __forceinline__ uint32_t lane_xor32(uint32_t v, int g) {
  const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // {upper <- lane - 32, lower <- lane + 32}
  return g ? sw[0] : sw[1];
}

template <int D>
__global__ void __launch_bounds__(256) elu1_bwd_kv16_kernel(Elu1BwdParams p) {
  constexpr int DC = D / 16, DT = D / 32;
  __shared__ __attribute__((aligned(1024))) bf16_t s_hi[D * D];
  __shared__ __attribute__((aligned(1024))) bf16_t s_lo[D * D];
  __shared__ float s_z[D];
  const int hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int64_t bh = (int64_t)b * p.n_heads + hs;
  const int n_groups = (p.Lkv + 31) / 32;
  const int g_end = min(n_groups, (blockIdx.x + 1) * p.kv_groups_per_wg);
  const bf16_t* kbase = (const bf16_t*)p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + g * 8;
  const bf16_t* vbase = (const bf16_t*)p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + g * 8;
  bf16x8 kf[DC], vf[DC];
  auto load_group = [&](int gi, bf16x8(&kd)[DC], bf16x8(&vd)[DC]) {
    const int t = gi * 32 + l32;
    const int64_t tr = t < p.Lkv ? t : 0;  // rows past the end re-read row 0; nothing is stored for them
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      kd[c] = *(const bf16x8*)(kbase + tr * p.k_st + c * 16);
      vd[c] = *(const bf16x8*)(vbase + tr * p.v_st + c * 16);
    }
  };
  int gi = blockIdx.x * p.kv_groups_per_wg + w;
  if (gi < g_end) load_group(gi, kf, vf);  // in flight while the state gradient is staged
  stage_hilo<D>(p.dstate + bh * D * D, s_hi, s_lo, tid);
  for (int e = tid; e < D; e += 256) s_z[e] = p.dz[bh * D + e];
  __syncthreads();
  bf16_t* dkb = (bf16_t*)p.dk + (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh;
  bf16_t* dvb = (bf16_t*)p.dv + (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh;
#pragma unroll 1
  for (; gi < g_end; gi += 4) {
    const int t = gi * 32 + l32;
    const bool ok = t < p.Lkv;
    bf16x8 pk[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pk[c][e] = (bf16_t)elu1f((float)kf[c][e]);
    }
    // k at this lane's epilogue channels 32 jt + 8 rq + 4 g + i lies in chunk 4 jt + rq, elements
    // 4g..: fragment c = 2 jt + rq / 2 of the lane half rq & 1. The two lanes of a token swap the
    // halves the other needs; afterwards kf[c] holds elements 4g.. of chunk 2c, then of chunk 2c + 1.
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const u32x4 u = __builtin_bit_cast(u32x4, kf[c]);
      const uint32_t m0 = g ? u[2] : u[0], m1 = g ? u[3] : u[1];  // own elements 4g..
      const uint32_t s0 = g ? u[0] : u[2], s1 = g ? u[1] : u[3];  // the partner's elements
      const uint32_t r0 = (uint32_t)__shfl_xor((int)s0, 32, 64), r1 = (uint32_t)__shfl_xor((int)s1, 32, 64);
      kf[c] = __builtin_bit_cast(bf16x8, g ? u32x4{r0, r1, m0, m1} : u32x4{m0, m1, r0, r1});
    }
#pragma unroll 1
    for (int jt = 0; jt < DT; ++jt) {
      f32x16 dk = f32x16{}, dv = f32x16{};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        dk = wa_mfma32(tile_tr8n<D>(s_hi, c, 32 * jt, lane), vf[c], dk);
        dk = wa_mfma32(tile_tr8n<D>(s_lo, c, 32 * jt, lane), vf[c], dk);
        dv = wa_mfma32(tile_row8<D>(s_hi, 32 * jt + l32, 2 * c + g), pk[c], dv);
        dv = wa_mfma32(tile_row8<D>(s_lo, 32 * jt + l32, 2 * c + g), pk[c], dv);
      }
      const bf16x8 k01[2] = {kf[0], kf[1]};  // this tile's K values (the array rotates below)
      // after the last column tile's products the fragments are dead: the next group's loads go out
      // before this tile's stores
      if (jt == DT - 1 && gi + 4 < g_end) load_group(gi + 4, kf, vf);
      // this lane's bf16 results: channels 32 jt + 8 rq + 4 g .. + 3 of its token, as two u32 each
      uint32_t ku[4][2], vu[4][2];
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int e0 = 32 * jt + 8 * rq + 4 * g;
        const f32x4 z4 = *(const f32x4*)(s_z + e0);
        const bf16x8 kc = k01[rq >> 1];  // fragments 2 jt, 2 jt + 1
        bf16x4 ok4, ov4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float kv = (float)kc[4 * (rq & 1) + i];
          ok4[i] = (bf16_t)((dk[rq * 4 + i] + z4[i]) * elu1_grad(kv));
          ov4[i] = (bf16_t)dv[rq * 4 + i];
        }
        const u32x2 k2 = __builtin_bit_cast(u32x2, ok4), v2 = __builtin_bit_cast(u32x2, ov4);
        ku[rq][0] = k2[0]; ku[rq][1] = k2[1];
        vu[rq][0] = v2[0]; vu[rq][1] = v2[1];
      }
      // The two lanes of a token swap halves so that each stores 16 bytes (8 consecutive channels):
      // of chunks 2 kk and 2 kk + 1, lane g keeps chunk 2 kk + g and sends its partner its own four
      // channels of chunk 2 kk + 1 - g. (Every lane swaps; only the store depends on the token.)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        uint32_t out_k[4], out_v[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t sk = g ? ku[2 * kk][j] : ku[2 * kk + 1][j], sv = g ? vu[2 * kk][j] : vu[2 * kk + 1][j];
          const uint32_t mk = g ? ku[2 * kk + 1][j] : ku[2 * kk][j], mv = g ? vu[2 * kk + 1][j] : vu[2 * kk][j];
          const uint32_t rk = lane_xor32(sk, g), rv = lane_xor32(sv, g);
          // channels 0..3 of the chunk come from the g = 0 lane, 4..7 from the g = 1 lane
          out_k[j] = g ? rk : mk;
          out_k[2 + j] = g ? mk : rk;
          out_v[j] = g ? rv : mv;
          out_v[2 + j] = g ? mv : rv;
        }
        if (ok) {
          const int e = 32 * jt + 8 * (2 * kk + g);
          *(u32x4*)(dkb + (int64_t)t * p.dk_st + e) = u32x4{out_k[0], out_k[1], out_k[2], out_k[3]};
          *(u32x4*)(dvb + (int64_t)t * p.dv_st + e) = u32x4{out_v[0], out_v[1], out_v[2], out_v[3]};
        }
      }
      // rotate so the next column tile's fragments sit at 0 and 1 (static register indices: a
      // runtime index into the array compiles to select chains)
      if (jt < DT - 1) {
#pragma unroll
        for (int c = 0; c + 2 < DC; ++c) kf[c] = kf[c + 2];
      }
    }
  }
}

// Key side at D = 128, bf16 K / V in and bf16 dK / dV out, streamed. Wave w owns output column
// tile w (32 channels) of both products for every token of the workgroup's run, with its operands
// of the state gradient (column slice for dK, row slice for dV, bf16 hi + lo: 32 fragments) read
// from LDS once into registers. K and V tiles of 32 tokens stream through a 3-stage LDS ring by
// direct-to-LDS loads, two tiles ahead; phi(K) is formed once per tile into LDS, and the results
// are staged in LDS and leave as whole 256-byte rows. Per tile a wave reads 16 KiB of B fragments
// for its 32 MFMAs (elu1_bwd_kv16_kernel reads 128 KiB of state fragments for 128) and waits on no
// load it issued itself. The fragments and their order are elu1_bwd_kv16_kernel's, so the results
// are bit-identical to it (and to elu1_bwd_kv_kernel rounded to bf16).
//
// Every step issues the same vector memory operations per thread: 4 tile loads (2 K, 2 V; past
// the run's last tile they read nothing, through an empty buffer range, into the stage just
// consumed) and 4 stores (2 dK, 2 dV; rows past Lkv fall outside the store's buffer range). Tile
// `it` is therefore waited for with a fixed count of younger operations (vector memory operations
// complete in issue order): after the loads of tile it come those of tiles it + 1 and it + 2 and
// the stores of the up to three steps before it.
template <int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) elu1_bwd_kvr_kernel(Elu1BwdParams p) {
  static_assert(D == 128, "one 32-channel column tile per wave");
  constexpr int DC = D / 16, TS = 32;
  constexpr int TILE = TS * D;               // bf16 elements of one K or V tile (8 KiB)
  constexpr int CPR = D / 8, RPI = 64 / CPR;  // 16-byte chunks per row, rows per wave instruction
  constexpr int NI = TS / (RPI * 4);          // instructions per wave per tensor and tile
  static_assert(NI == 2 && TS * CPR == 2 * 256, "fixed per-thread operation counts");
  // Stage s: K at 2s TILE, V at (2s + 1) TILE. While the state gradient's fragments are read, its
  // hi and lo tiles occupy TILEs 2-5 and 6-9; afterwards TILEs 2-5 are stages 1 and 2, TILE 6
  // phi(K), TILEs 7 and 8 the staged dK and dV rows.
  __shared__ __attribute__((aligned(1024))) bf16_t lds[10 * TILE];
  bf16_t* const s_hi = lds + 2 * TILE;
  bf16_t* const s_lo = lds + 6 * TILE;
  bf16_t* const pt = lds + 6 * TILE;
  bf16_t* const okt = lds + 7 * TILE;
  bf16_t* const ovt = lds + 8 * TILE;

  const int hs = blockIdx.y, b = blockIdx.z;
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bh = (int64_t)b * p.n_heads + hs;
  const int n_groups = (p.Lkv + TS - 1) / TS;
  const int g0 = blockIdx.x * p.kv_groups_per_wg;
  const int ntiles = min(n_groups, g0 + p.kv_groups_per_wg) - g0;
  const bf16_t* kbase = (const bf16_t*)p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16_t* vbase = (const bf16_t*)p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  bf16_t* dkbase = (bf16_t*)p.dk + (int64_t)b * p.dk_sb + (int64_t)h * p.dk_sh;
  bf16_t* dvbase = (bf16_t*)p.dv + (int64_t)b * p.dv_sb + (int64_t)h * p.dv_sh;

  // direct-to-LDS lane offsets: instruction i of wave w fills rows (4 i + w) RPI .. + RPI; lane L
  // writes row + L / CPR, slot L % CPR, which holds chunk slot ^ dual_swizzle(row)
  int k_off[NI], v_off[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int row = (4 * i + w) * RPI + lane / CPR, pos = lane % CPR;
    const int chunk = pos ^ dual_swizzle<D>(row);
    k_off[i] = (int)(row * p.k_st + chunk * 8) * 2;
    v_off[i] = (int)(row * p.v_st + chunk * 8) * 2;
  }
  auto issue = [&](int it, int s) {
    const bool real = it < ntiles;
    const int t0 = real ? (g0 + it) * TS : 0;
    const int rows = real ? min(TS, p.Lkv - t0) : 0;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kbase + (int64_t)t0 * p.k_st), (short)0, rows ? (int)((rows - 1) * p.k_st + D) * 2 : 0, WA_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vbase + (int64_t)t0 * p.v_st), (short)0, rows ? (int)((rows - 1) * p.v_st + D) * 2 : 0, WA_BUF_DWORD3);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int r0 = (4 * i + w) * RPI;
      lds_dma16(krs, lds + 2 * s * TILE + r0 * D, k_off[i]);
      lds_dma16(vrs, lds + (2 * s + 1) * TILE + r0 * D, v_off[i]);
    }
  };

  issue(0, 0);
  // z at this lane's epilogue channels 32 w + 8 rq + 4 g + i
  f32x4 zr[4];
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) zr[rq] = *(const f32x4*)(p.dz + bh * D + 32 * w + 8 * rq + 4 * g);
  stage_hilo<D>(p.dstate + bh * D * D, s_hi, s_lo, tid);
  __syncthreads();
  bf16x8 akh[DC], akl[DC], avh[DC], avl[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    akh[c] = tile_tr8n<D>(s_hi, c, 32 * w, lane);
    akl[c] = tile_tr8n<D>(s_lo, c, 32 * w, lane);
    avh[c] = tile_row8<D>(s_hi, 32 * w + l32, 2 * c + g);
    avl[c] = tile_row8<D>(s_lo, 32 * w + l32, 2 * c + g);
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave holds its fragments
  issue(1, 1);
  issue(2, 2);

  for (int it = 0; it < ntiles; ++it) {
    const int s = it % 3;
    const bf16_t* kt = lds + 2 * s * TILE;
    const bf16_t* vt = kt + TILE;
    // tile it has landed in every wave's share, and the previous step's reads are done
    if (it >= 3) asm volatile("s_waitcnt vmcnt(20)\n\ts_barrier" ::: "memory");
    else if (it == 2) asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
    else if (it == 1) asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    // phi(K) at the same swizzled positions (elementwise: a slot's chunk does not matter)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ci = tid + 256 * u, r = ci / CPR, pos = ci % CPR;
      bf16x8 x = *(const bf16x8*)(kt + r * D + pos * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (bf16_t)elu1f((float)x[e]);
      *(bf16x8*)(pt + r * D + pos * 8) = x;
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // dK^T[e, t] = sum_d dS^T[d, e] v[t, d], dV^T[d, t] = sum_e dS^T[d, e] phi(k)[t, e] (lane = token)
    f32x16 dk = f32x16{}, dv = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const bf16x8 vb = tile_row8<D>(vt, l32, 2 * c + g);
      const bf16x8 pb = tile_row8<D>(pt, l32, 2 * c + g);
      dk = wa_mfma32(akh[c], vb, dk);
      dk = wa_mfma32(akl[c], vb, dk);
      dv = wa_mfma32(avh[c], pb, dv);
      dv = wa_mfma32(avl[c], pb, dv);
    }
    // this lane's channels 32 w + 8 rq + 4 g + i of token l32, staged as 8-byte pieces
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int at = l32 * D + (((4 * w + rq) ^ dual_swizzle<D>(l32)) * 8) + 4 * g;
      const bf16x4 k4 = *(const bf16x4*)(kt + at);
      bf16x4 ok4, ov4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ok4[i] = (bf16_t)((dk[rq * 4 + i] + zr[rq][i]) * elu1_grad((float)k4[i]));
        ov4[i] = (bf16_t)dv[rq * 4 + i];
      }
      *(bf16x4*)(okt + at) = ok4;
      *(bf16x4*)(ovt + at) = ov4;
    }
    // staged rows complete; stage s is free for tile it + 3
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(it + 3, s);
    const int t0 = (g0 + it) * TS, rows = min(TS, p.Lkv - t0);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(dkbase + (int64_t)t0 * p.dk_st), (short)0, (int)((rows - 1) * p.dk_st + D) * 2, WA_BUF_DWORD3);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(dvbase + (int64_t)t0 * p.dv_st), (short)0, (int)((rows - 1) * p.dv_st + D) * 2, WA_BUF_DWORD3);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ci = tid + 256 * u, r = ci / CPR, cc = ci % CPR;
      const u32x4 ko = __builtin_bit_cast(u32x4, tile_row8<D>(okt, r, cc));
      const u32x4 vo = __builtin_bit_cast(u32x4, tile_row8<D>(ovt, r, cc));
      __builtin_amdgcn_raw_buffer_store_b128(ko, krs, (int)(r * p.dk_st + cc * 8) * 2, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(vo, vrs, (int)(r * p.dv_st + cc * 8) * 2, 0, 0);
    }
  }
  // the ring's last (empty) loads and the stores drain before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__global__ void __launch_bounds__(256) elu1_bwd_reduce_kernel(Elu1BwdParams p, int D) {
  const int64_t per = (int64_t)D * D + D;
  const int64_t total = (int64_t)p.B * p.n_heads * per;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  int c = 0;
  for (; c + 4 <= p.n_qt; c += 4) {
    a0 += p.part[(int64_t)c * total + i];
    a1 += p.part[(int64_t)(c + 1) * total + i];
    a2 += p.part[(int64_t)(c + 2) * total + i];
    a3 += p.part[(int64_t)(c + 3) * total + i];
  }
  for (; c < p.n_qt; ++c) a0 += p.part[(int64_t)c * total + i];
  const float s = (a0 + a1) + (a2 + a3);
  const int64_t bh = i / per, r = i % per;
  if (r < (int64_t)D * D) p.dstate[bh * D * D + r] = s;
  else p.dz[bh * D + (r - (int64_t)D * D)] = s;
}

int state_chunks(int64_t B, int64_t nh, int64_t L) {
  const int64_t target = 256;
  const int64_t per_bh = (target + B * nh - 1) / (B * nh);
  const int64_t max_chunks = (L + 63) / 64;
  const int64_t c = per_bh < max_chunks ? per_bh : max_chunks;
  return (int)(c < 1 ? 1 : c);
}

}  // namespace

extern "C" int64_t wa_elu1_state_workspace_bytes(int64_t B, int64_t n_heads, int64_t L, int64_t D) {
  const int64_t chunks = state_chunks(B, n_heads, L);
  return ((chunks * B * n_heads * (D * D + D)) * 4 + 255) / 256 * 256;
}

extern "C" int wa_elu1_state(const wa_elu1_state_args* a, void* stream) {
  WA_CHECK_ARG(a && a->k && a->v && a->state && a->zsum && a->workspace, "wa_elu1_state: null argument");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_elu1_state: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->dtype == WA_F32 || a->dtype == WA_BF16, "wa_elu1_state: bad dtype");
  WA_CHECK_ARG(a->L > 0 && a->H > 0 && a->B >= 0, "wa_elu1_state: bad sizes");
  const int64_t vec = a->dtype == WA_BF16 ? 8 : 4;
  WA_CHECK_ARG(wa_aligned16(a->k) && wa_aligned16(a->v) && a->k_sb % vec == 0 && a->k_st % vec == 0 &&
                   a->k_sh % vec == 0 && a->v_sb % vec == 0 && a->v_st % vec == 0 && a->v_sh % vec == 0,
               "wa_elu1_state: k/v must be 16-byte aligned with 16-byte aligned rows");
  WA_CHECK_ARG(a->L == 1 || (a->k_st >= a->D && a->v_st >= a->D && a->k_st < (1 << 24) && a->v_st < (1 << 24)),
               "wa_elu1_state: token strides must be at least D and below 2^24 elements");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || nh == 0) return WA_OK;
  StateParams sp{};
  sp.k = a->k; sp.k_sb = a->k_sb; sp.k_st = a->k_st; sp.k_sh = a->k_sh;
  sp.v = a->v; sp.v_sb = a->v_sb; sp.v_st = a->v_st; sp.v_sh = a->v_sh;
  sp.H = (int)a->H; sp.L = (int)a->L; sp.n_heads = (int)nh; sp.B = (int)a->B;
  sp.n_chunks = state_chunks(a->B, nh, a->L);
  sp.chunk_len = (int)(((a->L + sp.n_chunks - 1) / sp.n_chunks + 63) / 64 * 64);
  sp.n_chunks = (int)((a->L + sp.chunk_len - 1) / sp.chunk_len);
  sp.heads = a->heads; sp.part = (float*)a->workspace; sp.state = a->state; sp.zsum = a->zsum;
  dim3 grid((unsigned)sp.n_chunks, (unsigned)nh, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  if (a->D == 128) {
    if (a->dtype == WA_BF16) hipLaunchKernelGGL((elu1_state_dma_kernel<128, 8>), grid, dim3(512), 0, s, sp);
    else hipLaunchKernelGGL((elu1_state_kernel<128, float>), grid, dim3(256), 0, s, sp);
  } else {
    if (a->dtype == WA_BF16) hipLaunchKernelGGL((elu1_state_dma_kernel<64, 4>), grid, dim3(256), 0, s, sp);
    else hipLaunchKernelGGL((elu1_state_kernel<64, float>), grid, dim3(256), 0, s, sp);
  }
  int rc = wa_launch_status("elu1_state");
  if (rc != WA_OK) return rc;
  const int64_t total4 = a->B * nh * (a->D * a->D + a->D) / 4;
  hipLaunchKernelGGL(elu1_reduce_kernel, dim3((unsigned)((total4 + 63) / 64)), dim3(256), 0, s, sp, (int)a->D);
  return wa_launch_status("elu1_reduce");
}

extern "C" int wa_elu1_readout(const wa_elu1_readout_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->state && a->zsum && a->o, "wa_elu1_readout: null argument");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_elu1_readout: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->q_dtype == WA_F32 || a->q_dtype == WA_BF16, "wa_elu1_readout: bad q dtype");
  WA_CHECK_ARG(a->o_dtype == WA_F32 || a->o_dtype == WA_BF16, "wa_elu1_readout: bad o dtype");
  WA_CHECK_ARG(a->epilogue == WA_EPI_PLAIN || a->epilogue == WA_EPI_GATED, "wa_elu1_readout: epilogue must be PLAIN or GATED");
  WA_CHECK_ARG(wa_aligned16(a->state), "wa_elu1_readout: state must be 16-byte aligned");
  const int64_t vec = a->q_dtype == WA_BF16 ? 8 : 4;
  WA_CHECK_ARG(wa_aligned16(a->q) && a->q_sb % vec == 0 && a->q_st % vec == 0 && a->q_sh % vec == 0,
               "wa_elu1_readout: q must be 16-byte aligned with 16-byte aligned rows");
  WA_CHECK_ARG((((uintptr_t)a->o) & 7u) == 0 && a->o_sb % 4 == 0 && a->o_st % 4 == 0 && a->o_sh % 4 == 0,
               "wa_elu1_readout: output must be 8-byte aligned with strides multiple of 4");
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "wa_elu1_readout: gate_w must be 16-byte aligned");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || nh == 0 || a->L == 0) return WA_OK;
  ReadoutParams rp{a->q, a->q_sb, a->q_st, a->q_sh, a->q_dtype, a->state, a->zsum, a->o, a->o_sb, a->o_st,
                   a->o_sh, a->o_dtype, (int)a->H, (int)a->L, (int)nh, a->heads, a->epilogue,
                   (const bf16_t*)a->gate_w, a->gate_b, a->gate_pre_bf16, a->gate_out_bf16, a->lin_round_bf16};
  dim3 grid((unsigned)((a->L + 127) / 128), (unsigned)nh, (unsigned)a->B);
  hipStream_t s = (hipStream_t)stream;
  const bool hot = a->q_dtype == WA_BF16 && a->o_dtype == WA_BF16 && a->epilogue == WA_EPI_GATED && a->gate_w &&
                   a->gate_out_bf16 && a->lin_round_bf16;
  const int mode = hot ? (a->gate_pre_bf16 ? 1 : 2) : 0;
  if (a->D == 128) {
    if (mode == 1) hipLaunchKernelGGL((elu1_readout_kernel<128, 1>), grid, dim3(512), 0, s, rp);
    else if (mode == 2) hipLaunchKernelGGL((elu1_readout_kernel<128, 2>), grid, dim3(512), 0, s, rp);
    else hipLaunchKernelGGL((elu1_readout_kernel<128, 0>), grid, dim3(512), 0, s, rp);
  } else {
    if (mode == 1) hipLaunchKernelGGL((elu1_readout_kernel<64, 1>), grid, dim3(512), 0, s, rp);
    else if (mode == 2) hipLaunchKernelGGL((elu1_readout_kernel<64, 2>), grid, dim3(512), 0, s, rp);
    else hipLaunchKernelGGL((elu1_readout_kernel<64, 0>), grid, dim3(512), 0, s, rp);
  }
  return wa_launch_status("elu1_readout");
}

extern "C" int64_t wa_elu1_bwd_workspace_bytes(int64_t B, int64_t n_heads, int64_t Lq, int64_t D) {
  const int64_t nqt = (Lq + 127) / 128;
  return ((nqt * B * n_heads * (D * D + D) + B * n_heads * (D * D + D)) * 4 + 255) / 256 * 256;
}

extern "C" int wa_elu1_bwd(const wa_elu1_bwd_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->k && a->v && a->dout && a->state && a->zsum && a->workspace,
               "wa_elu1_bwd: null argument");
  WA_CHECK_ARG(a->dq && a->dk && a->dv, "wa_elu1_bwd: dq, dk and dv are required");
  WA_CHECK_ARG(a->dkv_dtype == WA_F32 || (a->dkv_dtype == WA_BF16 && !a->dk_accumulate && !a->dv_accumulate),
               "wa_elu1_bwd: dkv_dtype must be WA_F32, or WA_BF16 without accumulation");
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_elu1_bwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG((a->q_dtype == WA_F32 || a->q_dtype == WA_BF16) && (a->kv_dtype == WA_F32 || a->kv_dtype == WA_BF16) &&
                   (a->dout_dtype == WA_F32 || a->dout_dtype == WA_BF16),
               "wa_elu1_bwd: bad dtype");
  WA_CHECK_ARG(a->Lq > 0 && a->Lkv > 0 && a->H > 0 && a->B >= 0, "wa_elu1_bwd: bad sizes");
  const int64_t vq = a->q_dtype == WA_BF16 ? 8 : 4, vk = a->kv_dtype == WA_BF16 ? 8 : 4, vg = a->dout_dtype == WA_BF16 ? 8 : 4;
  WA_CHECK_ARG(wa_aligned16(a->q) && wa_aligned16(a->k) && wa_aligned16(a->v) && wa_aligned16(a->dout) &&
                   wa_aligned16(a->state) && wa_aligned16(a->workspace) && a->q_sb % vq == 0 && a->q_st % vq == 0 &&
                   a->q_sh % vq == 0 && a->k_sb % vk == 0 && a->k_st % vk == 0 && a->k_sh % vk == 0 &&
                   a->v_sb % vk == 0 && a->v_st % vk == 0 && a->v_sh % vk == 0 && a->d_sb % vg == 0 &&
                   a->d_st % vg == 0 && a->d_sh % vg == 0,
               "wa_elu1_bwd: tensors must be 16-byte aligned with 16-byte aligned rows");
  const int64_t nh = a->heads ? a->n_heads : a->H;
  if (a->B == 0 || nh == 0) return WA_OK;
  Elu1BwdParams bp{};
  bp.q = a->q; bp.q_sb = a->q_sb; bp.q_st = a->q_st; bp.q_sh = a->q_sh; bp.q_dtype = a->q_dtype;
  bp.k = a->k; bp.k_sb = a->k_sb; bp.k_st = a->k_st; bp.k_sh = a->k_sh;
  bp.v = a->v; bp.v_sb = a->v_sb; bp.v_st = a->v_st; bp.v_sh = a->v_sh; bp.kv_dtype = a->kv_dtype;
  bp.g = a->dout; bp.g_sb = a->d_sb; bp.g_st = a->d_st; bp.g_sh = a->d_sh; bp.g_dtype = a->dout_dtype;
  bp.state = a->state; bp.zsum = a->zsum;
  bp.dq = a->dq; bp.dq_sb = a->dq_sb; bp.dq_st = a->dq_st; bp.dq_sh = a->dq_sh; bp.dq_acc = a->dq_accumulate;
  bp.dk = a->dk; bp.dk_sb = a->dk_sb; bp.dk_st = a->dk_st; bp.dk_sh = a->dk_sh; bp.dk_acc = a->dk_accumulate;
  bp.dv = a->dv; bp.dv_sb = a->dv_sb; bp.dv_st = a->dv_st; bp.dv_sh = a->dv_sh; bp.dv_acc = a->dv_accumulate;
  bp.dkv_bf16 = a->dkv_dtype == WA_BF16;
  bp.heads = a->heads; bp.n_heads = (int)nh; bp.H = (int)a->H; bp.B = (int)a->B; bp.Lq = (int)a->Lq;
  bp.Lkv = (int)a->Lkv; bp.n_qt = (int)((a->Lq + 127) / 128);
  bp.part = (float*)a->workspace;
  bp.dstate = bp.part + (int64_t)bp.n_qt * a->B * nh * (a->D * a->D + a->D);
  bp.dz = bp.dstate + a->B * nh * a->D * a->D;
  hipStream_t s = (hipStream_t)stream;
  dim3 gq((unsigned)bp.n_qt, (unsigned)nh, (unsigned)a->B), gk((unsigned)((a->Lkv + 127) / 128), (unsigned)nh, (unsigned)a->B);
  const int64_t total = a->B * nh * (a->D * a->D + a->D);
  int rc;
  if (a->D == 128) hipLaunchKernelGGL(elu1_bwd_q_kernel<128>, gq, dim3(512), 0, s, bp);
  else hipLaunchKernelGGL(elu1_bwd_q_kernel<64>, gq, dim3(512), 0, s, bp);
  if ((rc = wa_launch_status("elu1_bwd_q"))) return rc;
  hipLaunchKernelGGL(elu1_bwd_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, bp, (int)a->D);
  if ((rc = wa_launch_status("elu1_bwd_reduce"))) return rc;
  // bf16 K / V and bf16 dK / dV with 16-byte aligned rows: the streaming kernel
  const bool kv16 = bp.dkv_bf16 && a->kv_dtype == WA_BF16 && wa_aligned16(a->dk) && wa_aligned16(a->dv) &&
                    a->dk_sb % 8 == 0 && a->dk_st % 8 == 0 && a->dk_sh % 8 == 0 && a->dv_sb % 8 == 0 &&
                    a->dv_st % 8 == 0 && a->dv_sh % 8 == 0;
  if (kv16) {
    // about two workgroups per CU (64 KB of staged state each at D = 128), each staging the state
    // gradient once for its run of 32-token groups
    const int64_t n_groups = (a->Lkv + 31) / 32;
    const int64_t per_bh = std::max<int64_t>(1, std::min<int64_t>((n_groups + 3) / 4, (512 + a->B * nh - 1) / (a->B * nh)));
    bp.kv_groups_per_wg = (int)((n_groups + per_bh - 1) / per_bh);
    const dim3 gk16((unsigned)((n_groups + bp.kv_groups_per_wg - 1) / bp.kv_groups_per_wg), (unsigned)nh, (unsigned)a->B);
    // the streamed kernel addresses a 32-token tile's rows with 32-bit byte offsets
    const bool streamed = a->D == 128 && a->k_st < (1 << 24) && a->v_st < (1 << 24) && a->dk_st < (1 << 24) &&
                          a->dv_st < (1 << 24) && a->k_st >= a->D && a->v_st >= a->D && a->dk_st >= a->D &&
                          a->dv_st >= a->D;
    if (streamed) hipLaunchKernelGGL(elu1_bwd_kvr_kernel<128>, gk16, dim3(256), 0, s, bp);
    else if (a->D == 128) hipLaunchKernelGGL(elu1_bwd_kv16_kernel<128>, gk16, dim3(256), 0, s, bp);
    else hipLaunchKernelGGL(elu1_bwd_kv16_kernel<64>, gk16, dim3(256), 0, s, bp);
  } else {
    if (a->D == 128) hipLaunchKernelGGL(elu1_bwd_kv_kernel<128>, gk, dim3(256), 0, s, bp);
    else hipLaunchKernelGGL(elu1_bwd_kv_kernel<64>, gk, dim3(256), 0, s, bp);
  }
  return wa_launch_status("elu1_bwd_kv");
}
