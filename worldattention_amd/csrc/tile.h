// LDS tile helpers shared by the attention backward kernels (gfx950).
//
// A "step tile" is 64 rows x D bf16 (one 64-key or 64-query slice), stored row-major in LDS with
// an XOR swizzle on its 16-byte chunks. The backward kernels read every tile both ways:
//   * 128-bit reads (ds_read_b128) of one chunk of 16 consecutive rows: gfx950 serves 16 lanes
//     (256 bytes, all 64 banks) per cycle;
//   * transpose reads (ds_read_b64_tr_b16) of 4 consecutive rows x 32 bytes per 16 lanes.
// dual_swizzle<D> keeps both conflict-free: it is injective over any 16 consecutive rows (per row
// parity for D = 64, whose 128-byte rows share a bank line in pairs), and rows r, r+1, r+2, r+3
// (r aligned to 4) differ in the swizzle bits above bit 0, so a transpose read's 8 chunk halves
// land in 8 distinct chunk pairs.
#pragma once
#include "common.h"

typedef short wa_s16x4 __attribute__((ext_vector_type(4)));
#define WA_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
#define WA_LDS_S16X4(p) ((__attribute__((address_space(3))) wa_s16x4*)(p))

template <int D>
__device__ __forceinline__ int dual_swizzle(int r) {
  return D == 128 ? (2 * (r & 3)) | (8 * ((r >> 2) & 1)) | ((r >> 3) & 1)
                  : (2 * ((r >> 1) & 1)) | (4 * ((r >> 2) & 1)) | ((r >> 3) & 1);
}

// One direct-to-LDS wave instruction of a step-tile stream: instruction i of wave w (NW waves)
// writes rows r0 = (i NW + w) RPI .. +RPI (1 KiB), lane L row r0 + L / CPR, slot L % CPR, which
// holds chunk slot ^ dual_swizzle(row). Rows at or past `real` re-read the tile's row 0 (in-bounds,
// finite data that the caller masks).
template <int D, int NW>
__device__ __forceinline__ void tile_dma_one(bf16_t* lds, const bf16_t* tile, int64_t st, int real, int w,
                                             int lane, int i) {
  constexpr int CPR = D / 8;
  constexpr int RPI = 64 / CPR;
  const int rin = lane / CPR, pos = lane % CPR;
  const int r0 = (i * NW + w) * RPI;
  const int row = r0 + rin;
  const int chunk = pos ^ dual_swizzle<D>(row);
  const int src = row < real ? row : 0;
  __builtin_amdgcn_global_load_lds((const void*)(tile + (int64_t)src * st + chunk * 8), WA_LDS_PTR(lds + r0 * D),
                                   16, 0, 0);
}

template <int D, int NW>
__device__ __forceinline__ void tile_dma(bf16_t* lds, const bf16_t* tile, int64_t st, int real, int w, int lane) {
  constexpr int NI = 64 / ((64 / (D / 8)) * NW);
#pragma unroll
  for (int i = 0; i < NI; ++i) tile_dma_one<D, NW>(lds, tile, st, real, w, lane, i);
}

// 128-bit fragment: row `row`, chunk `chunk` (8 bf16) of a swizzled tile.
template <int D>
__device__ __forceinline__ bf16x8 tile_row8(const bf16_t* lds, int row, int chunk) {
  return *(const bf16x8*)(lds + row * D + ((chunk ^ dual_swizzle<D>(row)) * 8));
}

// Transpose-read fragment for an MFMA operand whose contraction runs over 16 tile rows of chunk
// c with the accumulator-order permutation K(c, g, e) = 16c + 4g + 8(e / 4) + e % 4, at column
// col0 + l32 (lane = (l32, g)). This is the order in which a 32x32 accumulator's registers 8h..8h+7
// hold their rows, so probabilities / gradients feed the next product straight from registers.
// Transpose-read semantics (per 16-lane group): result lane i, element r comes from element i % 4
// of source lane 4r + i / 4.
template <int D>
__device__ __forceinline__ bf16x8 tile_tr8(const bf16_t* lds, int c, int col0, int lane) {
  const int G = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
  bf16x8 a;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int row = 16 * c + 4 * (G >> 1) + 8 * hf + r;
    const int col = col0 + 16 * (G & 1) + 4 * q;
    const int slot = (col >> 3) ^ dual_swizzle<D>(row);
    const wa_s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(WA_LDS_S16X4(lds + row * D + slot * 8 + (col & 7)));
    const bf16x4 b = __builtin_bit_cast(bf16x4, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[4 * hf + e] = b[e];
  }
  return a;
}

// Transpose-read fragment in natural contraction order: lane (l32, g) receives rows
// 16c + 8g + e (e = 0..7) at column col0 + l32.
template <int D>
__device__ __forceinline__ bf16x8 tile_tr8n(const bf16_t* lds, int c, int col0, int lane) {
  const int G = lane >> 4, r = (lane & 15) >> 2, q = lane & 3;
  bf16x8 a;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int row = 16 * c + 8 * (G >> 1) + 4 * hf + r;
    const int col = col0 + 16 * (G & 1) + 4 * q;
    const int slot = (col >> 3) ^ dual_swizzle<D>(row);
    const wa_s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(WA_LDS_S16X4(lds + row * D + slot * 8 + (col & 7)));
    const bf16x4 b = __builtin_bit_cast(bf16x4, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) a[4 * hf + e] = b[e];
  }
  return a;
}

// Stores 8 consecutive bf16 of row `row`, chunk `chunk` into a dual-swizzled tile.
template <int D>
__device__ __forceinline__ void tile_put8(bf16_t* lds, int row, int chunk, const bf16x8& v) {
  *(bf16x8*)(lds + row * D + ((chunk ^ dual_swizzle<D>(row)) * 8)) = v;
}
