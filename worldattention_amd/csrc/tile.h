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

// Direct-to-LDS buffer loads written as inline assembly (16 or 4 bytes per lane; lane L writes LDS
// at `lds` + 16 L or + 4 L). The compiler neither sees nor tracks these loads, so its own wait
// insertion never stalls an LDS read behind them; every kernel that uses them orders them itself
// with s_waitcnt vmcnt + s_barrier. (Through the builtins, the compiler makes some reads of one
// ring stage wait for the loads in flight into the others.)
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
  const unsigned m0 = (unsigned)(size_t)WA_LDS_PTR(lds);
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
}
// The same from a 64-bit per-lane global address (no buffer descriptor, no 32-bit offset limit).
__device__ __forceinline__ void lds_dma16_global(const void* src, void* lds) {
  const unsigned m0 = (unsigned)(size_t)WA_LDS_PTR(lds);
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
// The same with device-scope coherence (sc1): reads data another XCD wrote with sc1 stores.
__device__ __forceinline__ void lds_dma16_sc1(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
  const unsigned m0 = (unsigned)(size_t)WA_LDS_PTR(lds);
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
  const unsigned m0 = (unsigned)(size_t)WA_LDS_PTR(lds);
  asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(m0) : "memory");
}

// A step-tile stream over one slab (rows 0 .. R-1 with row stride `st` elements, `slab_bytes`
// from the first row's start to the last row's end) by direct-to-LDS buffer loads. Instruction i
// of wave w fills rows r0 = (i NW + w) RPI .. +RPI (1 KiB): lane L row r0 + L / CPR, slot L % CPR,
// which holds chunk slot ^ dual_swizzle(row). Each tile gets a descriptor that starts at its
// first row and ends at the slab's end, so the buffer range check (on the per-lane offset) turns
// rows past the slab into zeros; the per-lane offsets are loop-invariant.
template <int D, int NW>
struct TileStream {
  static constexpr int CPR = D / 8;           // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per wave instruction
  static constexpr int NI = 64 / (RPI * NW);  // instructions per wave per tile
  const char* base;
  int64_t st_bytes, slab_bytes;
  int off[NI];
  __device__ __forceinline__ void init(const bf16_t* b, int64_t st, int64_t slab, int w, int lane) {
    base = (const char*)b;
    st_bytes = st * 2;
    slab_bytes = slab;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (i * NW + w) * RPI + lane / CPR, pos = lane % CPR;
      off[i] = (int)(row * st_bytes) + (pos ^ dual_swizzle<D>(row)) * 16;
    }
  }
  // rows row0 .. row0 + 63 (row0 < R, uniform) into `lds`
  __device__ __forceinline__ void issue(bf16_t* lds, int row0, int w) const {
    const int64_t o = (int64_t)row0 * st_bytes;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + o), (short)0, (int)(slab_bytes - o), WA_BUF_DWORD3);
#pragma unroll
    for (int i = 0; i < NI; ++i)
      lds_dma16(rs, lds + (i * NW + w) * RPI * D, off[i]);
  }
};

// 64 consecutive fp32 values (lane L: element first + L; past `count` elements: zero) into `lds`
// by one direct-to-LDS buffer load per wave.
__device__ __forceinline__ void row_stats_dma(float* lds, const float* first, int count, int lane) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)first, (short)0, count * 4, WA_BUF_DWORD3);
  lds_dma4(rs, lds, lane * 4);
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
