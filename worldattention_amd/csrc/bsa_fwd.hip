// Block-sparse flash-attention forward for gfx950 (bf16 MFMA 32x32x16, fp32 accumulation).
//
// Work decomposition. A "row" is one (batch, head, query block) with its list of key blocks
// index[b,h,i,0:num]. A row's list is cut into up to max_splits units of at most `split` visits;
// one workgroup processes one (row, split) unit. A row with one unit writes its output directly.
// The units of a longer row write a normalized partial output plus its log2-sum-exp to the
// workspace and count their arrival on a per-row counter; the last unit to arrive merges every
// partial in split order, applies the fusion epilogue and writes the row, so every result is
// independent of scheduling (one launch, no merge kernel).
//
// Unit kernel (one workgroup = BS/32 waves; wave w owns query rows [32w, 32w+32) of the block).
// Per visited key block the K and V tiles are streamed global -> LDS with direct-to-LDS loads
// (no register staging), into two separate buffers so that the next K tile streams in while the
// softmax and the PV product of the current one run. Products use the transposed formulation
//     S^T[key, q] = K[key, :] . Q[q, :]         (A = K from LDS, B = Q^T in registers)
//     O^T[d, q]  += V^T[d, key] . P^T[key, q]   (A = V^T by transpose-reads of row-major V)
// so each lane owns one query column: the row max / row sum need one exchange with lane^32 and
// the probabilities feed the PV product straight from the QK accumulator registers.
//
// LDS layouts (no padding; XOR swizzles on 16-byte chunks keep every read conflict-free):
//   K[key][chunk ^ (key & 15)]      read with ds_read_b128 (16 lanes = 16 keys, one chunk; D = 128)
//   V[key][chunk ^ 2*(key & 3)]      read with ds_read_b64_tr_b16 (16 lanes = 4 keys x 32 bytes)
//
// Reference semantics: wan/modules/hsa/block_sparse_triton.py:67-139 (online softmax, partial
// trailing block mask, empty list -> 0, LSE output) and block_sparse_torch.py:16-64 (id clamping,
// listed order, duplicates attended twice, fp32 math).
#include <mutex>

#include "common.h"
#include "tile.h"

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define WA_LDS(p) ((__attribute__((address_space(3))) void*)(p))
#define WA_LDS4(p) ((__attribute__((address_space(3))) s16x4*)(p))

struct FwdParams {
  const bf16_t* q; int64_t q_sb, q_st, q_sh;
  const bf16_t* k; int64_t k_sb, k_st, k_sh;
  const bf16_t* v; int64_t v_sb, v_st, v_sh;
  void* o; int64_t o_sb, o_st, o_sh; int o_dtype;
  float* lse;
  const int32_t* index; const int32_t* num; int64_t index_width;
  const int32_t* block_sizes;
  const int32_t* heads; int n_heads;
  int B, H, Lq, Lkv, Nq, Nkv;
  float scale_log2;
  int epilogue;
  const void* x; int64_t x_sb, x_st, x_sh; int x_dtype;
  const bf16_t* gate_w; const float* gate_b;
  int gate_pre_bf16, gate_out_bf16, attn_round_bf16;
  // split bookkeeping
  const int32_t* units;  // [n_units][2] = (row, split) or NULL: unit u = (u / max_splits, u % max_splits)
  int n_units, max_splits, split;
  int64_t n_rows;
  int k_slab_bytes, v_slab_bytes;  // bytes of one (batch, head) K / V slab: rows 0 .. Lkv-1
  float* part_o;         // [rows * max_splits][BS][D] normalized partial outputs
  float* part_lse;       // [rows * max_splits][BS] log2-sum-exp of the partials
  int* arrivals;         // [rows] units of the row done so far (zeroed by the launch)
};

// Workgroup barrier without the global-memory fence of __syncthreads (which would wait for the
// in-flight K/V tile loads). LDS reads before it have completed: their results were consumed.
__device__ __forceinline__ void wa_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// `irow` numbers rows by global head, (b * H + h) * Nq + i: the layout of index / num. Units and
// workspace slots number rows by head slot instead, (b * n_heads + slot) * Nq + i.
__device__ __forceinline__ int row_visits(const FwdParams& p, int64_t irow) {
  if (!p.index) return p.Nkv;
  const int n = p.num[irow];
  return max(0, min(n, (int)p.index_width));
}

// Ascending bitonic sort of one int per lane across the 64-lane wave.
__device__ __forceinline__ int wave_sort_ascending(int key, int lane) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int other = __shfl_xor(key, j, 64);
      const bool keep_min = ((lane & j) == 0) == ((lane & k) == 0);
      key = keep_min ? min(key, other) : max(key, other);
    }
  }
  return key;
}

__device__ __forceinline__ int block_real(const FwdParams& p, int j, int BS) {
  int real = BS;
  if (p.block_sizes) real = min(real, p.block_sizes[j]);
  real = min(real, p.Lkv - j * BS);
  return max(real, 0);
}

// 16-byte chunk swizzles. gfx950 serves a 128-bit LDS read 16 lanes (256 bytes, all 64 banks)
// per cycle, and the transpose read 16 lanes x 8 bytes (128 bytes) per cycle:
//   K row r, D = 128 (256-byte rows): chunk ^ (r & 15) — 16 consecutive keys hit 16 distinct
//     chunk slots of their rows, i.e. all 64 banks;
//   K row r, D = 64 (128-byte rows, two per bank line): chunk ^ ((r >> 1) & 7);
//   V row r: chunk ^ 2 (r & 3) — a transpose read's 16 lanes cover 4 rows x 32 bytes, which this
//     spreads over 4 x 8 distinct banks.
template <int D>
__device__ __forceinline__ int k_swizzle(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
__device__ __forceinline__ int v_swizzle(int r) { return 2 * (r & 3); }

// One [64, D] bf16 step tile (64 consecutive key rows) streamed into swizzled LDS with
// direct-to-LDS buffer loads. Wave instruction i moves 1 KiB = RPI whole rows: lane L writes row
// r0(i) + L / CPR, slot L % CPR, and so reads the chunk that the swizzle stores in that slot. The
// per-lane byte offsets within a tile are loop-invariant; a tile is selected by its buffer
// descriptor, which starts at the tile's first row and ends at the slab's end. Rows past a partial
// block's end read either the following keys (finite, masked or multiplied by a zero probability)
// or, past the slab, zeros.
template <int D, int NW>
struct NextTile {
  static constexpr int CPR = D / 8;                  // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;               // rows per wave instruction (4 or 8)
  static constexpr int NI = 64 / (RPI * NW);         // instructions per wave per tensor
  __amdgpu_buffer_rsrc_t k_rs, v_rs;                 // start at the tile's first row; empty past the list
  bf16_t* k_lds; bf16_t* v_lds;
  int k_off[NI], v_off[NI];                          // this lane's byte offset per instruction
  __device__ __forceinline__ void k(int i, int w, int) const {
    if (i < NI) lds_dma16(k_rs, k_lds + (i * NW + w) * RPI * D, k_off[i]);
  }
  __device__ __forceinline__ void v(int i, int w, int) const {
    if (i < NI) lds_dma16(v_rs, v_lds + (i * NW + w) * RPI * D, v_off[i]);
  }
};

// Writes one query column's result (lane = query qi, accumulator layout d = 32t + 8(r/4) + 4g +
// r%4) with the fusion epilogue:
//   PLAIN: o = attn;  FUSE: o = attn + g * x;  GATED: o = g * attn,
// g = sigmoid(q . gate_w[d] + gate_b[d]) (or sigmoid(q) without gate_w): the gated fusion of
// attention.py:246-254, in registers.
template <int D>
__device__ __forceinline__ void write_output(const FwdParams& p, const f32x16 (&acc)[D / 32], float inv,
                                             const bf16x8 (&qf)[D / 16], const bf16_t* qrow, int b, int h,
                                             int qi, bool q_ok, int g, int l32) {
  constexpr int DC = D / 16, DT = D / 32;
  const int epilogue = p.epilogue;
  const bool need_gate = epilogue != WA_EPI_PLAIN;
  f32x16 gacc[DT];
  if (need_gate && p.gate_w) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      // the tile's gate rows in one round trip (left to itself the scheduler waited for each)
      bf16x8 a[DC];
#pragma unroll
      for (int c = 0; c < DC; ++c) a[c] = *(const bf16x8*)(p.gate_w + (t * 32 + l32) * D + c * 16 + g * 8);
#pragma unroll
      for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(a[c]));
      gacc[t] = f32x16{};
#pragma unroll
      for (int c = 0; c < DC; ++c) gacc[t] = wa_mfma32(a[c], qf[c], gacc[t]);
    }
  }
  if (!q_ok) return;
  // Per 32-channel tile every global read (gate bias, q, the fused input x) is issued before the
  // tile's stores: a store may alias a later read, which would otherwise cost one memory round
  // trip per element.
  const int64_t xo = (int64_t)b * p.x_sb + (int64_t)qi * p.x_st + (int64_t)h * p.x_sh;
  const int64_t oo = (int64_t)b * p.o_sb + (int64_t)qi * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    float pre[4][4], xv[4][4];
    if (need_gate) {
      // The options branch around whole tiles and the tile's loads are all issued before the first
      // use (with the options tested per element, every element waited for its own load).
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = t * 32 + 8 * rq + 4 * g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (p.gate_w) pre[rq][i] = p.gate_b ? p.gate_b[d0 + i] : 0.f;
          else pre[rq][i] = (float)qrow[d0 + i];
        }
      }
      if (epilogue == WA_EPI_FUSE && p.x_dtype == WA_BF16) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[rq][i] = (float)((const bf16_t*)p.x)[xo + t * 32 + 8 * rq + 4 * g + i];
      } else if (epilogue == WA_EPI_FUSE) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[rq][i] = ((const float*)p.x)[xo + t * 32 + 8 * rq + 4 * g + i];
      } else {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
#pragma unroll
          for (int i = 0; i < 4; ++i) xv[rq][i] = 0.f;
      }
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(pre[rq][i]), "+v"(xv[rq][i]));
      if (p.gate_w) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
#pragma unroll
          for (int i = 0; i < 4; ++i) pre[rq][i] = gacc[t][rq * 4 + i] + pre[rq][i];
      }
    }
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int d0 = t * 32 + 8 * rq + 4 * g;
      float val[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = acc[t][rq * 4 + i] * inv;
        if (p.attn_round_bf16) a = wa_bf16_round(a);
        if (need_gate) {
          float pr = pre[rq][i];
          if (p.gate_pre_bf16) pr = wa_bf16_round(pr);
          float gs = wa_sigmoid(pr);
          if (p.gate_out_bf16) gs = wa_bf16_round(gs);
          a = epilogue == WA_EPI_FUSE ? wa_add_rn(a, wa_mul_rn(xv[rq][i], gs)) : wa_mul_rn(a, gs);
        }
        val[i] = a;
      }
      if (p.o_dtype == WA_BF16) {
        bf16x4 ov = {(bf16_t)val[0], (bf16_t)val[1], (bf16_t)val[2], (bf16_t)val[3]};
        *(bf16x4*)((bf16_t*)p.o + oo + d0) = ov;
      } else {
        f32x4 ov = {val[0], val[1], val[2], val[3]};
        *(f32x4*)((float*)p.o + oo + d0) = ov;
      }
    }
  }
}

// Step cursor over the unit's visits: a visit of a BS = 128 block is two 64-key steps (the second
// only when the block has more than 64 real keys), of a BS = 64 block one step. All fields are
// wave-uniform.
struct Cursor {
  uint64_t todo;  // visits not yet started (bit = lane holding the visit)
  int j, real;    // current block and its real key count
  int half;       // current 64-key step within the block
  bool valid;
};

template <int BS>
__device__ __forceinline__ void cursor_next(Cursor& c, int my_j, int my_real) {
  if (BS == 128 && c.valid && c.half == 0 && c.real > 64) {
    c.half = 1;
    return;
  }
  if (c.todo) {
    const int v = __builtin_ctzll(c.todo);
    c.todo &= c.todo - 1;
    c.j = __builtin_amdgcn_readlane(my_j, v);
    c.real = __builtin_amdgcn_readlane(my_real, v);
    c.half = 0;
    c.valid = true;
  } else {
    c.valid = false;
  }
}

// One 64-key step of the online softmax on LDS buffer (kb, vb): S^T = K Q^T, lazily rescaled
// exponentials, O^T += V^T P^T. `real` = real keys of this step (1..64). The next step's tile
// stream (`nt`) is issued in slices between the products.
template <int D, int NW>
__device__ __forceinline__ void attend_step(const bf16_t* kb, const bf16_t* vb, const int (&k_rd)[D / 16],
                                            const int (&v_rd)[2], const bf16x8 (&qf)[D / 16],
                                            f32x16 (&oacc)[D / 32], float& m_i, float& l_i, int real, int g,
                                            float scale_log2, const NextTile<D, NW>& nt, int w, int lane) {
  constexpr int KT = 2, DC = D / 16, DT = D / 32, PC = 4;
  constexpr int NI = NextTile<D, NW>::NI;
  f32x16 sacc[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) sacc[kt] = f32x16{};
  bf16x8 ka[KT], kn[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) ka[kt] = *(const bf16x8*)(kb + k_rd[0] + kt * 32 * D);
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    if (c + 1 < DC) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) kn[kt] = *(const bf16x8*)(kb + k_rd[c + 1] + kt * 32 * D);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) sacc[kt] = wa_mfma32(ka[kt], qf[c], sacc[kt]);
    if (c % (DC / NI > 0 ? DC / NI : 1) == 0) nt.k(c / (DC / NI > 0 ? DC / NI : 1), w, lane);
    if (c + 1 < DC) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) ka[kt] = kn[kt];
    }
  }
  if (DC < NI) {
#pragma unroll
    for (int i = DC; i < NI; ++i) nt.k(i, w, lane);
  }
  if (real < 64) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key >= real) sacc[kt][r] = -INFINITY;
      }
    }
  }
  // Exponentials against the running max m_i, which may lag the scores: the step is accepted when
  // every lane's sum of exponentials is at most 2^16 (so is each exponential: far from fp32 / bf16
  // overflow). Otherwise (the first step, or scores more than ~11 above m_i) m_i moves to the step
  // max, the accumulators are rescaled and the exponentials recomputed. The final normalization
  // uses the same m_i, so the result does not depend on how far m_i lags.
  float rs;
  bf16x8 pb[PC];
  auto exps = [&]() {
    rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[kt][r], scale_log2, -m_i));
        rs += pv;
        pb[kt * 2 + (r >> 3)][r & 7] = (bf16_t)pv;
      }
    }
  };
  exps();
  if (__any(!(rs <= 65536.f))) {
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    }
    // every step has a real key, so mx is finite; on the first step m_i = -inf and alpha = 0
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
    const float m_new = fmaxf(mx, m_i);
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
    l_i *= alpha;
    m_i = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] *= alpha;
    exps();
  }
  l_i += rs;
  // V of this step: everything but the next step's K slices (the last NI loads) has landed, and
  // after the barrier every wave's has.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NI) : "memory");
#pragma unroll
  for (int c = 0; c < PC; ++c) {
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      bf16x8 a;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const s16x4 vv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            WA_LDS4(vb + v_rd[t & 1] + (16 * c + 8 * hf) * D + (t >> 1) * 64));
        const bf16x4 vb4 = __builtin_bit_cast(bf16x4, vv);
#pragma unroll
        for (int e = 0; e < 4; ++e) a[4 * hf + e] = vb4[e];
      }
      oacc[t] = wa_mfma32(a, pb[c], oacc[t]);
    }
    if (NI >= PC) {
#pragma unroll
      for (int i = c * (NI / PC); i < (c + 1) * (NI / PC); ++i) nt.v(i, w, lane);
    } else if (c < NI) {
      nt.v(c, w, lane);
    }
  }
}

template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) __attribute__((amdgpu_waves_per_eu(2)))
bsa_unit_kernel(FwdParams p) {
  constexpr int NW = BS / 32;   // waves; wave w owns query rows [32w, 32w + 32)
  constexpr int DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D;  // elements of one K (or V) step tile
  // Two K and two V step tiles (64 KiB at D = 128: two workgroups per CU), fed by inline-assembly
  // direct-to-LDS loads that the compiler does not track (the kernel orders them itself).
  __shared__ __attribute__((aligned(1024))) bf16_t kr[2 * TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t vr[2 * TILE];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;

  const int u = wa_xcd_remap(blockIdx.x, p.n_units);
  // The prologue's memory reads in two round trips: the unit entry with the head map beside it,
  // then (once the row is known) its visit count, its list window and Q together.
  const int hmap = p.heads && lane < min(p.n_heads, 64) ? p.heads[lane] : 0;
  int64_t row;
  int split;
  if (p.units) {
    row = p.units[2 * u];
    split = p.units[2 * u + 1];
  } else {
    row = u / p.max_splits;
    split = u % p.max_splits;
  }
  if (row < 0 || row >= p.n_rows || split < 0 || split >= p.max_splits) return;
  const int qb = (int)(row % p.Nq);
  const int64_t bh = row / p.Nq;
  const int hs = (int)(bh % p.n_heads), b = (int)(bh / p.n_heads);
  int h = hs;
  if (p.heads) h = p.n_heads <= 64 ? __builtin_amdgcn_readlane(hmap, hs) : p.heads[hs];
  if (h < 0 || h >= p.H) return;  // uniform per workgroup
  const int64_t irow = ((int64_t)b * p.H + h) * p.Nq + qb;

  // The row's list entries at positions lane (j0) and split * p.split + lane (j1), read before its
  // visit count is known (in bounds of the row's index_width entries); the count then picks one.
  const int nraw = p.index ? p.num[irow] : p.Nkv;
  int j0 = 0, j1 = 0;
  if (p.index) {
    const int32_t* lrow = p.index + irow * p.index_width;
    if (lane < min((int)p.index_width, 64)) j0 = lrow[lane];
    const int lo1 = split * p.split;
    if (split > 0 && lane < min((int)p.index_width - lo1, 64)) j1 = lrow[lo1 + lane];
  }
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  // Q^T fragments (B operand): lane holds Q[qi, 16c + 8g .. +8).
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok ? qi : 0) * p.q_st;
  bf16x8 qf[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    bf16x8 t = *(const bf16x8*)(qrow + c * 16 + g * 8);
    qf[c] = q_ok ? t : bf16x8{};
  }

  const int n = p.index ? max(0, min(nraw, (int)p.index_width)) : nraw;
  const int s_begin = split * p.split;
  const int s_end = min(n, s_begin + p.split);
  // A unit beyond this row's list returns; split 0 of a row with no visits runs on with an empty
  // list and writes the empty row (zero attention).
  if (s_begin >= s_end && (n > 0 || split > 0)) return;
  const int ns = min((n + p.split - 1) / p.split, p.max_splits);
  const bf16_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;

  // List entries one per lane, read once: the loop fetches them with readlane and issues no memory
  // reads besides the tile streams. A row of at most 64 visits is loaded whole and sorted by block
  // id, and split s of the row's ns units takes the sorted positions s, s + ns, s + 2 ns, ...: every
  // unit of a head (they run together on one XCD) then sweeps the whole key range in step with the
  // others, so the units that list a block fetch it at about the same time and share it in L2.
  // The visit order only changes the summation order. Longer rows keep list order, one contiguous
  // slice per unit.
  const bool whole = n <= 64;
  const int lo = whole ? 0 : s_begin;
  const int take = whole ? n : s_end - s_begin;
  int my_j = 0;
  if (lane < take) my_j = p.index ? min(max(lo == 0 ? j0 : j1, 0), p.Nkv - 1) : lo + lane;
  if (whole) my_j = wave_sort_ascending(lane < take ? my_j : 0x7fffffff, lane);
  const bool mine = whole ? lane < n && lane % ns == split : lane < take;
  const int my_real = mine ? block_real(p, my_j, BS) : 0;
  Cursor cur{__ballot(mine && my_real > 0), 0, 0, 0, false};
  cursor_next<BS>(cur, my_j, my_real);

  // tile streams: this lane's loop-invariant chunk offsets; each tile gets a buffer descriptor that
  // starts at its first row and ends at the slab's end (rows past the slab read zeros), and a
  // step past the end of the list an empty one (zeros, no memory traffic)
  using NT = NextTile<D, NW>;
  int k_off[NT::NI], v_off[NT::NI];
#pragma unroll
  for (int i = 0; i < NT::NI; ++i) {
    const int row = (i * NW + w) * NT::RPI + lane / NT::CPR, pos = lane % NT::CPR;
    k_off[i] = (int)(row * p.k_st + (pos ^ k_swizzle<D>(row)) * 8) * 2;
    v_off[i] = (int)(row * p.v_st + (pos ^ v_swizzle(row)) * 8) * 2;
  }
  auto tile_rs = [&](const Cursor& c, bool is_k) {
    const bf16_t* base = is_k ? kbase : vbase;
    int64_t off = 0;
    int bytes = 0;
    if (c.valid) {
      off = (int64_t)(c.j * BS + 64 * c.half) * (is_k ? p.k_st : p.v_st);
      bytes = (is_k ? p.k_slab_bytes : p.v_slab_bytes) - (int)(off * 2);
    }
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, bytes, WA_BUF_DWORD3);
  };
  auto tiles = [&](bf16_t* kl, const Cursor& ck, bf16_t* vl, const Cursor& cv) {
    NT nt;
    nt.k_rs = tile_rs(ck, true);
    nt.v_rs = tile_rs(cv, false);
    nt.k_lds = kl;
    nt.v_lds = vl;
#pragma unroll
    for (int i = 0; i < NT::NI; ++i) {
      nt.k_off[i] = k_off[i];
      nt.v_off[i] = v_off[i];
    }
    return nt;
  };
  // Q fragments in registers before the first tile loads (a later first use would wait for them)
#pragma unroll
  for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[c]));
  // cursor of step t + 1; prologue K(0), V(0)
  Cursor c1 = cur;
  cursor_next<BS>(c1, my_j, my_real);
  if (cur.valid) {
    const NT a = tiles(kr, cur, vr, cur);
#pragma unroll
    for (int i = 0; i < NT::NI; ++i) a.k(i, w, lane);
#pragma unroll
    for (int i = 0; i < NT::NI; ++i) a.v(i, w, lane);
  }

  // Per-lane LDS read offsets (elements). K (A operand of S^T = K Q^T): lane reads row kt*32 + l32,
  // chunk 2c + g, stored in slot (2c + g) ^ k_swizzle(l32) (the swizzle of kt*32 + l32 equals
  // that of l32).
  int k_rd[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_rd[c] = l32 * D + ((2 * c + g) ^ k_swizzle<D>(l32)) * 8;
  // V (A operand of O^T += V^T P^T via transpose reads): 16-lane group G, source lane j = 4r + q
  // reads 4 elements of row 16c + 4(G/2) + 8hf + r at column 32t + 16(G%2) + 4q, whose chunk is
  // swizzled by 2r: 8 (t / 2) + ((4 (t % 2) + 2 (G % 2) + q / 2) ^ 2r).
  const int G = lane >> 4, tr_r = (lane & 15) >> 2, tr_q = lane & 3;
  int v_rd[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
    v_rd[t] = (4 * (G >> 1) + tr_r) * D + (((4 * t + 2 * (G & 1) + (tr_q >> 1)) ^ (2 * tr_r)) * 8) + 4 * (tr_q & 1);

  f32x16 oacc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
  float m_i = -INFINITY, l_i = 0.f;

  // Step t computes on K(t), V(t) in stage t % 2; its QK product streams K(t + 1) and its PV
  // product V(t + 1) into the other stage. At the top of step t only V(t) may still be in flight
  // (the last NI loads), and before the PV product (attend_step) only K(t + 1); the barriers extend
  // each wave's wait to the workgroup and order a stage's refill after every wave's reads of it.
  // Two steps per iteration (stage 0, then stage 1), so every LDS address is a loop-invariant
  // register plus an immediate offset.
  while (cur.valid) {
#pragma unroll
    for (int vs = 0; vs < 2; ++vs) {
      if (!cur.valid) break;
      const int real = cur.real - 64 * cur.half;
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NT::NI) : "memory");
      attend_step<D, NW>(kr + vs * TILE, vr + vs * TILE, k_rd, v_rd, qf, oacc, m_i, l_i, real, g, p.scale_log2,
                         tiles(kr + (vs ^ 1) * TILE, c1, vr + (vs ^ 1) * TILE, c1), w, lane);
      cur = c1;
      cursor_next<BS>(c1, my_j, my_real);
    }
  }

  // the last steps streamed empty tiles: let them land before the workgroup's LDS is freed
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const float lsum = l_i + __shfl_xor(l_i, 32, 64);
  float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  // log2-sum-exp of this unit's keys; the row's natural-log lse is this times ln 2
  float lse2 = lsum > 0.f ? m_i + __log2f(lsum) : -INFINITY;
  if (ns > 1) {
    // Normalized partial + log2-sum-exp; the row's last unit to arrive merges every partial, in
    // split order (its own is still in registers: the same fp32 values it stored). The row's units
    // may run on different XCDs, whose L2s are not coherent with each other, so the partials are
    // written and read with device-scope (sc1) buffer accesses instead of L2-wide write-back and
    // invalidate, and the arrival count is a device-scope atomic taken after this workgroup's
    // partial stores have completed; the last arrival loads the others' partials only after its
    // count has returned. A partial is stored in accumulator-fragment order (wave, tile, quad,
    // lane), so every store and load instruction covers 1 KiB of contiguous memory.
    const int64_t slot0 = row * p.max_splits;
    const int ql = w * 32 + l32;
    constexpr int SLOT_BYTES = BS * D * 4;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.part_o + slot0 * (BS * D)), (short)0, ns * SLOT_BYTES, WA_BUF_DWORD3);
    auto frag_off = [&](int sp, int t, int rq) { return sp * SLOT_BYTES + (((w * DT + t) * 4 + rq) * 64 + lane) * 16; };
    constexpr int SC1 = 16;  // cache policy: device-scope coherent
    if (g == 0)
      __hip_atomic_store(p.part_lse + (slot0 + split) * BS + ql, lse2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const f32x4 ov = {oacc[t][rq * 4] * inv, oacc[t][rq * 4 + 1] * inv, oacc[t][rq * 4 + 2] * inv,
                          oacc[t][rq * 4 + 3] * inv};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ov), prs, frag_off(split, t, rq), 0, SC1);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* s_last = (int*)kr;  // the K ring is free: every tile load has landed and been read
    if (tid == 0) {
      const bool last =
          __hip_atomic_fetch_add(p.arrivals + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ns - 1;
      if (last) __hip_atomic_store(p.arrivals + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // reusable
      *s_last = last;
    }
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(*s_last)) return;  // uniform: one LDS word for every lane
    // Another unit's partial comes in by direct-to-LDS loads into this wave's 16 KiB of the free
    // K/V rings (each wave reads back only what it loaded: no workgroup barrier), the first one
    // together with the first four log2-sum-exps, so a two-unit row merges after one round trip.
    float* plse = p.part_lse + slot0 * BS + ql;
    auto load_lse = [&](int sp) {
      return sp == split ? lse2 : __hip_atomic_load(plse + sp * BS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    constexpr int WPH = (NW + 1) / 2;  // waves staged in each ring
    static_assert(WPH * DT * 4 * 1024 <= 2 * TILE * 2, "partial staging does not fit the rings");
    char* wbuf = (w < WPH ? (char*)kr : (char*)vr) + (w % WPH) * (DT * 4 * 1024);
    auto fetch_part = [&](int sp) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) lds_dma16_sc1(prs, wbuf + (t * 4 + rq) * 1024, frag_off(sp, t, rq));
      }
    };
    const int sp_first = split == 0 ? 1 : 0;
    fetch_part(sp_first);
    const float l0 = load_lse(0), l1 = load_lse(1);
    const float l2 = ns > 2 ? load_lse(2) : -INFINITY, l3 = ns > 3 ? load_lse(3) : -INFINITY;
    auto lse_of = [&](int sp) { return sp == 0 ? l0 : sp == 1 ? l1 : sp == 2 ? l2 : sp == 3 ? l3 : load_lse(sp); };
    float M = -INFINITY;
#pragma unroll 1
    for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, lse_of(sp));
    float Z = 0.f;
    if (M != -INFINITY) {
#pragma unroll 1
      for (int sp = 0; sp < ns; ++sp) {
        const float wgt = exp2f(lse_of(sp) - M);
        if (wgt != 0.f) Z += wgt;
      }
    }
    // sum the weighted partials in split order (zero weights skipped)
    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
#pragma unroll 1
    for (int sp = 0; sp < ns; ++sp) {
      const float wgt = M != -INFINITY ? exp2f(lse_of(sp) - M) : 0.f;
      if (sp == split) {
        if (wgt != 0.f) {
#pragma unroll
          for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[t][i] = fmaf(wgt, oacc[t][i] * inv, acc[t][i]);
          }
        }
        continue;
      }
      if (sp != sp_first) fetch_part(sp);  // the buffer is free: the previous partial was read
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (wgt != 0.f) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const f32x4 v = *(const f32x4*)(wbuf + (t * 4 + rq) * 1024 + lane * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][rq * 4 + i] = fmaf(wgt, v[i], acc[t][rq * 4 + i]);
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next fetch
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = acc[t];
    inv = Z > 0.f ? 1.f / Z : 0.f;
    lse2 = Z > 0.f ? M + log2f(Z) : -INFINITY;
  }
  if (p.lse && g == 0 && q_ok) p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = lse2 * WA_LN2;
  write_output<D>(p, oacc, inv, qf, qrow, b, h, qi, q_ok, g, l32);
}

// Merges the ns normalized partials of one row (slot = row * max_splits + split), in split order,
// and writes the row's output and lse; ns = 0 writes an empty row (no visits: zero attention).
template <int D, int BS>
__device__ __forceinline__ void merge_row(const FwdParams& p, int64_t row, int ns, int b, int h, int qb, int w, int lane) {
  constexpr int DC = D / 16, DT = D / 32;
  const int g = lane >> 5, l32 = lane & 31;
  const int qi = qb * BS + w * 32 + l32;
  const bool q_ok = qi < p.Lq;
  const int ql = w * 32 + l32;
  const int64_t slot0 = row * p.max_splits;

  float M = -INFINITY;
#pragma unroll 1
  for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, p.part_lse[(slot0 + sp) * BS + ql]);
  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float Z = 0.f;
  if (M != -INFINITY) {
#pragma unroll 1
    for (int sp = 0; sp < ns; ++sp) {
      const float ls = p.part_lse[(slot0 + sp) * BS + ql];
      const float wgt = exp2f(ls - M);
      if (wgt == 0.f) continue;
      Z += wgt;
      const float* po = p.part_o + (slot0 + sp) * (int64_t)(BS * D) + ql * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 v = *(const f32x4*)(po + t * 32 + 8 * rq + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][rq * 4 + i] = fmaf(wgt, v[i], acc[t][rq * 4 + i]);
        }
      }
    }
  }
  const float inv = Z > 0.f ? 1.f / Z : 0.f;
  if (p.lse && g == 0 && q_ok)
    p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = Z > 0.f ? (M + log2f(Z)) * WA_LN2 : -INFINITY;
  const bf16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok ? qi : 0) * p.q_st;
  bf16x8 qf[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    bf16x8 t = *(const bf16x8*)(qrow + c * 16 + g * 8);
    qf[c] = q_ok ? t : bf16x8{};
  }
  write_output<D>(p, acc, inv, qf, qrow, b, h, qi, q_ok, g, l32);
}

// Writes every row when there is no unit to launch (all rows empty).
template <int D, int BS>
__global__ void __launch_bounds__(2 * BS) bsa_empty_rows_kernel(FwdParams p) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row = blockIdx.x;
  const int qb = (int)(row % p.Nq);
  const int64_t bh = row / p.Nq;
  const int hs = (int)(bh % p.n_heads), b = (int)(bh / p.n_heads);
  const int h = p.heads ? p.heads[hs] : hs;
  if (h < 0 || h >= p.H) return;
  merge_row<D, BS>(p, row, 0, b, h, qb, w, lane);
}

__global__ void __launch_bounds__(256) bsa_clear_arrivals_kernel(int* arrivals, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) arrivals[i] = 0;
}

template <int D, int BS>
int launch(const FwdParams& fp, int64_t rows, bool cleared, hipStream_t stream) {
  if (!cleared) {
    hipLaunchKernelGGL(bsa_clear_arrivals_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream,
                       fp.arrivals, rows);
    const int rc = wa_launch_status("bsa_fwd_clear");
    if (rc != WA_OK) return rc;
  }
  hipLaunchKernelGGL((bsa_unit_kernel<D, BS>), dim3(fp.n_units), dim3(2 * BS), 0, stream, fp);
  return wa_launch_status("bsa_fwd_unit");
}

// Workspace layout: the split partials (fp32 [rows * max_splits][BS][D] outputs, then
// [rows * max_splits][BS] log2-sum-exps; only when a row can take more than one unit), then the
// int32 arrival counters [rows], each region starting on a 256-byte boundary.
int64_t partial_bytes(int64_t rows, int64_t max_splits, int64_t block_size, int64_t D) {
  return max_splits > 1 ? (rows * max_splits * block_size * (D + 1) * 4 + 255) / 256 * 256 : 0;
}

int64_t max_splits_of(int64_t max_visits, int64_t split) {
  return max_visits > 0 ? (max_visits + split - 1) / split : 1;
}

int bsa_fwd_impl(const wa_bsa_fwd_args* a, void* workspace, void* stream);

}  // namespace

extern "C" int64_t wa_bsa_fwd_workspace_bytes(int64_t rows, int64_t max_visits, int64_t split, int64_t block_size,
                                              int64_t D) {
  if (split <= 0) split = WA_BSA_DEFAULT_SPLIT;
  return partial_bytes(rows, max_splits_of(max_visits, split), block_size, D) + (rows * 4 + 255) / 256 * 256;
}

extern "C" int wa_bsa_fwd(const wa_bsa_fwd_args* a, void* stream) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_fwd: null args");
  return bsa_fwd_impl(a, a->workspace, stream);
}

// ---------------------------------------------------------------------------------------------
// wa_bsa_fwd_noalloc: the same launch with its workspace in a static device array of this library
// (one copy per GPU, allocated when the library's code is loaded on that GPU), for callers that
// cannot allocate device memory. The array's host-side name only stands for the symbol: its device
// address is looked up once per device with hipGetSymbolAddress and used from then on.
// ---------------------------------------------------------------------------------------------
namespace {

static __device__ __align__(256) unsigned char scratch[WA_BSA_FWD_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device that runs `stream` (the current device for the null
// stream), looked up on the first call for that device with the device current.
int scratch_address(void* stream, void** out) {
  int cur = 0;
  WA_CHECK_HIP(hipGetDevice(&cur));
  int dev = cur;
  if (stream) WA_CHECK_HIP(hipStreamGetDevice((hipStream_t)stream, &dev));
  WA_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "wa_bsa_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur) WA_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) WA_CHECK_HIP(hipSetDevice(cur));
    if (e != hipSuccess || p == nullptr)
      return wa_fail(e != hipSuccess ? (int)e : WA_ERR_UNSUPPORTED, "wa_bsa_fwd_noalloc: hipGetSymbolAddress: %s",
                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WA_OK;
}

}  // namespace

extern "C" int wa_bsa_fwd_noalloc(const wa_bsa_fwd_args* a, void* stream) {
  WA_CHECK_ARG(a != nullptr, "wa_bsa_fwd_noalloc: null args");
  WA_CHECK_ARG(a->workspace == nullptr && a->arrivals == nullptr,
               "wa_bsa_fwd_noalloc: workspace and arrivals must be NULL (the static scratch array holds both)");
  WA_CHECK_ARG(a->D > 0 && a->block_size > 0 && a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0,
               "wa_bsa_fwd_noalloc: bad sizes");
  const int64_t nq = (a->Lq + a->block_size - 1) / a->block_size;
  const int64_t nkv = (a->Lkv + a->block_size - 1) / a->block_size;
  const int64_t nh = a->heads ? a->n_heads : a->H;
  const int64_t rows = a->B * nh * nq;
  const int64_t split = a->split_visits > 0 ? a->split_visits : WA_BSA_DEFAULT_SPLIT;
  const int64_t width = a->index ? a->index_width : nkv;
  const int64_t max_visits = a->max_visits > 0 ? (a->max_visits < width ? a->max_visits : width) : width;
  const int64_t need = wa_bsa_fwd_workspace_bytes(rows, max_visits, split, a->block_size, a->D);
  WA_CHECK_ARG(need <= (int64_t)WA_BSA_FWD_NOALLOC_SCRATCH_BYTES,
               "wa_bsa_fwd_noalloc: the launch needs %lld bytes of workspace, more than the %lld-byte static "
               "scratch array; call wa_bsa_fwd with a workspace instead",
               (long long)need, (long long)WA_BSA_FWD_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(stream, &ws);
  if (rc != WA_OK) return rc;
  // arrivals == NULL: the launch clears the counters in the scratch array with a fill kernel first
  return bsa_fwd_impl(a, ws, stream);
}

namespace {

int bsa_fwd_impl(const wa_bsa_fwd_args* a, void* workspace, void* stream) {
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_bsa_fwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_bsa_fwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0, "wa_bsa_fwd: bad sizes");
  WA_CHECK_ARG(a->q && a->k && a->v && a->o, "wa_bsa_fwd: null tensor");
  WA_CHECK_ARG(workspace, "wa_bsa_fwd: workspace required (wa_bsa_fwd_workspace_bytes)");
  WA_CHECK_ARG(wa_aligned16(a->q) && wa_aligned16(a->k) && wa_aligned16(a->v) && wa_aligned16(workspace),
               "wa_bsa_fwd: q/k/v/workspace must be 16-byte aligned");
  WA_CHECK_ARG(a->q_sb % 8 == 0 && a->q_st % 8 == 0 && a->q_sh % 8 == 0 && a->k_sb % 8 == 0 &&
                   a->k_st % 8 == 0 && a->k_sh % 8 == 0 && a->v_sb % 8 == 0 && a->v_st % 8 == 0 &&
                   a->v_sh % 8 == 0,
               "wa_bsa_fwd: q/k/v strides must be multiples of 8 elements");
  WA_CHECK_ARG(a->o_dtype == WA_F32 || a->o_dtype == WA_BF16, "wa_bsa_fwd: bad output dtype");
  const uintptr_t oal = a->o_dtype == WA_F32 ? 15u : 7u;
  WA_CHECK_ARG((((uintptr_t)a->o) & oal) == 0 && a->o_sb % 4 == 0 && a->o_st % 4 == 0 && a->o_sh % 4 == 0,
               "wa_bsa_fwd: output must be 4-element aligned with strides multiple of 4");
  WA_CHECK_ARG(a->epilogue >= WA_EPI_PLAIN && a->epilogue <= WA_EPI_GATED, "wa_bsa_fwd: bad epilogue");
  if (a->epilogue == WA_EPI_FUSE)
    WA_CHECK_ARG(a->x && (a->x_dtype == WA_F32 || a->x_dtype == WA_BF16), "wa_bsa_fwd: FUSE needs x");
  if (a->gate_w) WA_CHECK_ARG(wa_aligned16(a->gate_w), "wa_bsa_fwd: gate_w must be 16-byte aligned");
  if (a->index) WA_CHECK_ARG(a->num && a->index_width > 0, "wa_bsa_fwd: index needs num and width");
  const int64_t nq = (a->Lq + a->block_size - 1) / a->block_size;
  const int64_t nkv = (a->Lkv + a->block_size - 1) / a->block_size;
  WA_CHECK_ARG(a->heads != nullptr || a->n_heads == 0, "wa_bsa_fwd: n_heads = %lld without a heads list",
               (long long)a->n_heads);
  const int64_t nh = a->heads ? a->n_heads : a->H;
  WA_CHECK_ARG(nh >= 0 && nh <= a->H, "wa_bsa_fwd: bad head count");
  const int64_t rows = a->B * nh * nq;
  const int64_t split = a->split_visits > 0 ? a->split_visits : WA_BSA_DEFAULT_SPLIT;
  WA_CHECK_ARG(split <= 64 && (a->block_size == 64 || split <= 32),
               "wa_bsa_fwd: split_visits %lld exceeds %d", (long long)split, a->block_size == 64 ? 64 : 32);
  const int64_t width = a->index ? a->index_width : nkv;
  const int64_t max_visits = a->max_visits > 0 ? (a->max_visits < width ? a->max_visits : width) : width;
  const int64_t max_splits = max_visits > 0 ? (max_visits + split - 1) / split : 1;
  const int64_t n_units = a->units ? a->n_units : rows * max_splits;
  WA_CHECK_ARG(rows < (int64_t)1 << 31 && n_units < (int64_t)1 << 31 && rows * max_splits < (int64_t)1 << 40 &&
                   a->Lq < (int64_t)1 << 30 && a->Lkv < (int64_t)1 << 30,
               "wa_bsa_fwd: problem too large");
  WA_CHECK_ARG(a->units == nullptr || a->n_units >= 0, "wa_bsa_fwd: bad unit count");
  if (rows == 0) return WA_OK;

  FwdParams fp{};
  fp.q = (const bf16_t*)a->q; fp.q_sb = a->q_sb; fp.q_st = a->q_st; fp.q_sh = a->q_sh;
  fp.k = (const bf16_t*)a->k; fp.k_sb = a->k_sb; fp.k_st = a->k_st; fp.k_sh = a->k_sh;
  fp.v = (const bf16_t*)a->v; fp.v_sb = a->v_sb; fp.v_st = a->v_st; fp.v_sh = a->v_sh;
  fp.o = a->o; fp.o_sb = a->o_sb; fp.o_st = a->o_st; fp.o_sh = a->o_sh; fp.o_dtype = a->o_dtype;
  fp.lse = a->lse;
  fp.index = a->index; fp.num = a->num; fp.index_width = a->index_width;
  fp.block_sizes = a->block_sizes;
  fp.heads = a->heads; fp.n_heads = (int)nh;
  fp.B = (int)a->B; fp.H = (int)a->H; fp.Lq = (int)a->Lq; fp.Lkv = (int)a->Lkv;
  fp.Nq = (int)nq; fp.Nkv = (int)nkv;
  const float scale = a->scale > 0.f ? a->scale : 1.0f / sqrtf((float)a->D);
  fp.scale_log2 = scale * WA_LOG2E;
  fp.epilogue = a->epilogue;
  fp.x = a->x; fp.x_sb = a->x_sb; fp.x_st = a->x_st; fp.x_sh = a->x_sh; fp.x_dtype = a->x_dtype;
  fp.gate_w = (const bf16_t*)a->gate_w; fp.gate_b = a->gate_b;
  fp.gate_pre_bf16 = a->gate_pre_bf16; fp.gate_out_bf16 = a->gate_out_bf16;
  fp.attn_round_bf16 = a->attn_round_bf16;
  fp.units = a->units; fp.n_units = (int)n_units; fp.max_splits = (int)max_splits; fp.split = (int)split;
  fp.n_rows = rows;
  // the tile streams address one (batch, head) slab with 32-bit byte offsets
  const int64_t k_slab = ((a->Lkv - 1) * a->k_st + a->D) * 2, v_slab = ((a->Lkv - 1) * a->v_st + a->D) * 2;
  WA_CHECK_ARG(k_slab < ((int64_t)1 << 31) && v_slab < ((int64_t)1 << 31) &&
                   ((int64_t)((a->Lkv + a->block_size - 1) / a->block_size) * a->block_size) * a->k_st * 2 < ((int64_t)1 << 31) &&
                   ((int64_t)((a->Lkv + a->block_size - 1) / a->block_size) * a->block_size) * a->v_st * 2 < ((int64_t)1 << 31),
               "wa_bsa_fwd: one K/V head slab must span less than 2 GiB");
  fp.k_slab_bytes = (int)k_slab;
  fp.v_slab_bytes = (int)v_slab;
  fp.part_o = (float*)workspace;
  fp.part_lse = fp.part_o + rows * max_splits * a->block_size * a->D;
  fp.arrivals = a->arrivals ? a->arrivals
                            : (int*)((char*)workspace + partial_bytes(rows, max_splits, a->block_size, a->D));
  const bool cleared = a->arrivals != nullptr;
  if (n_units == 0) fp.n_units = 0;

  hipStream_t s = (hipStream_t)stream;
  if (fp.n_units == 0) {
    // nothing to visit: every row is written as an empty row
    hipLaunchKernelGGL((a->D == 64 ? (a->block_size == 64 ? bsa_empty_rows_kernel<64, 64> : bsa_empty_rows_kernel<64, 128>)
                                   : (a->block_size == 64 ? bsa_empty_rows_kernel<128, 64> : bsa_empty_rows_kernel<128, 128>)),
                       dim3((unsigned)rows), dim3(2 * a->block_size), 0, s, fp);
    return wa_launch_status("bsa_fwd_empty_rows");
  }
  if (a->D == 64 && a->block_size == 64) return launch<64, 64>(fp, rows, cleared, s);
  if (a->D == 64 && a->block_size == 128) return launch<64, 128>(fp, rows, cleared, s);
  if (a->D == 128 && a->block_size == 64) return launch<128, 64>(fp, rows, cleared, s);
  return launch<128, 128>(fp, rows, cleared, s);
}

}  // namespace
