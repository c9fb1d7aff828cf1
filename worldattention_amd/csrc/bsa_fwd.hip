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
// The visited key blocks are 64-key steps whose K and V tiles stream global -> LDS with
// direct-to-LDS loads (no register staging) into two stages per tensor. Products use the
// transposed formulation
//     S^T[key, q] = K[key, :] . Q[q, :]         (A = K from LDS, B = Q^T in registers)
//     O^T[d, q]  += V^T[d, key] . P^T[key, q]   (A = V^T by transpose-reads of row-major V)
// so each lane owns one query column: the row max / row sum need one exchange with lane^32 and
// the probabilities feed the PV product straight from the QK accumulator registers. The step loop
// is software-pipelined in 32-key halves: each slot interleaves the softmax of one half with the
// QK product of the next and the PV product of the previous one inside the wave.
//
// LDS layouts (no padding; XOR swizzles on 16-byte chunks):
//   K[key][chunk ^ (key & 15)]      read with ds_read_b128 (16 lanes = 16 keys, one chunk; D = 128)
//   V[key][chunk ^ 2*(key & 3)]      read with ds_read_b64_tr_b16 (16 lanes = 4 keys x 32 bytes)
// Each 16-lane read phase touches distinct chunk slots, but the counters still see bank conflicts:
// 1.3 conflict cycles per LDS instruction in the kernel before the pipelined loop.
//
// Reference semantics: wan/modules/hsa/block_sparse_triton.py:67-139 (online softmax, partial
// trailing block mask, empty list -> 0, LSE output) and block_sparse_torch.py:16-64 (id clamping,
// listed order, duplicates attended twice, fp32 math).
#include <mutex>
#include <type_traits>

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

// ---------------------------------------------------------------------------------------------
// Software-pipelined step loop. A 64-key step is two 32-key halves, and the loop runs in "slots",
// one half each. Slot (block b, half h) does three independent pieces of work:
//   * the softmax of the half-step whose scores the previous slot produced: S[1 - h] -> the
//     probability chunks P[2(1-h)], P[2(1-h)+1] and the slot's row sum;
//   * the QK product of half h of step b (K stage of step b) -> S[h];
//   * the PV product of half h of step b - 1 (V stage of step b - 1) with P[2h], P[2h+1];
// plus, in the block's first slot, the tile loads of the next block (K of step b + 1, V of step b:
// both stages were last read in block b - 1, so the loads go out a whole block ahead). The softmax (~56 VALU instructions at D = 128)
// interleaves with the 16 products inside the wave, so the SIMD issues VALU work while the MFMA
// pipe is busy instead of after it.
// ---------------------------------------------------------------------------------------------

// Direct-to-LDS 16-byte load through the compiler's builtin: the scheduler sees a memory load (LDS
// reads move freely around it) and the wait-count pass tracks it per LDS array. Every ring stage is
// an array of its own and every access names its stage statically, so a read of one stage never
// waits for loads into another; the kernel still orders loads across waves itself (s_waitcnt
// vmcnt(0) + s_barrier at the top of each block).
__device__ __forceinline__ void pipe_dma16(__amdgpu_buffer_rsrc_t rs, bf16_t* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Instruction-group order of one slot: after a few leading LDS reads, each product is followed by
// up to DSN LDS reads and VAN VALU instructions, and every VMEVERY-th product by one tile load.
template <int I, int N, int DSN, int VAN, int VMEVERY>
__device__ __forceinline__ void pipe_sched() {
  if constexpr (I < N) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, DSN, 0);  // LDS read
    __builtin_amdgcn_sched_group_barrier(0x002, VAN, 0);  // VALU
    if constexpr (VMEVERY > 0 && I % VMEVERY == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
    pipe_sched<I + 1, N, DSN, VAN, VMEVERY>();
  }
}

// Tile loads of one slot: NI direct-to-LDS loads of a tensor's next tile into stage `lds`.
struct PipeLoad {
  __amdgpu_buffer_rsrc_t rs;
  bf16_t* lds;
};

// One slot (see above) of a wave that owns QT 32-query tiles. SMH: half whose softmax runs (1 - the
// product half). SM / QK / PV / LD switch the pieces on for the pipeline's first and last blocks.
// With QT = 2 every K and V fragment read from LDS feeds two products. rs[qt]: the slot's row sum
// of exponentials of tile qt (this lane's 16 keys).
template <int D, int NW, int QT, int SMH, bool SM, bool QK, bool PV, bool LD, int KROW = -1>
__device__ __forceinline__ void pipe_slot(f32x16 (&S)[2][QT], bf16x8 (&P)[4][QT], f32x16 (&oacc)[QT][D / 32],
                                          const bf16x8 (&qf)[QT][D / 16], const bf16_t* kst, const bf16_t* vst,
                                          const int (&k_rd)[D / 16], const int (&v_rd)[2], const float (&neg_m)[QT],
                                          float scale_log2, const PipeLoad& ldk, const int (&koff)[NextTile<D, NW>::NI],
                                          const PipeLoad& ldv, const int (&voff)[NextTile<D, NW>::NI], int w,
                                          float (&rs)[QT]) {
  constexpr int H = SMH ^ 1, DC = D / 16, DT = D / 32;
  constexpr int RH = KROW < 0 ? H : KROW;  // key half of the K / V rows (the key-split loop fixes it)
  constexpr int NI = NextTile<D, NW>::NI, RPI = NextTile<D, NW>::RPI;
  // operands from LDS: K rows 32 RH + l32 (A of S^T = K Q^T), V^T of keys 32 RH .. +32 (A of O^T += V^T P^T)
  bf16x8 kf[DC];
  if constexpr (QK) {
#pragma unroll
    for (int c = 0; c < DC; ++c) kf[c] = *(const bf16x8*)(kst + k_rd[c] + RH * 32 * D);
  }
  bf16x8 vf[2][DT];
  if constexpr (PV) {
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const s16x4 vv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              WA_LDS4(vst + v_rd[t & 1] + (16 * (2 * RH + cc) + 8 * hf) * D + (t >> 1) * 64));
          const bf16x4 vb4 = __builtin_bit_cast(bf16x4, vv);
#pragma unroll
          for (int e = 0; e < 4; ++e) vf[cc][t][4 * hf + e] = vb4[e];
        }
      }
    }
  }
  if constexpr (QK) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) S[H][qt] = wa_mfma32(kf[0], qf[qt][0], f32x16{});
#pragma unroll
    for (int c = 1; c < DC; ++c) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) S[H][qt] = wa_mfma32(kf[c], qf[qt][c], S[H][qt]);
    }
  }
  if constexpr (PV) {
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) oacc[qt][t] = wa_mfma32(vf[cc][t], P[2 * H + cc][qt], oacc[qt][t]);
      }
    }
  }
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) rs[qt] = 0.f;
  if constexpr (SM) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float r0 = 0.f, r1 = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(S[SMH][qt][r], scale_log2, neg_m[qt]));
        if (r & 1) r1 += pv;
        else r0 += pv;
        P[2 * SMH + (r >> 3)][qt][r & 7] = (bf16_t)pv;
      }
      rs[qt] = r0 + r1;
    }
  }
  if constexpr (LD) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      pipe_dma16(ldk.rs, ldk.lds + (i * NW + w) * RPI * D, koff[i]);
      pipe_dma16(ldv.rs, ldv.lds + (i * NW + w) * RPI * D, voff[i]);
    }
  }
  constexpr int NM = QT * ((QK ? DC : 0) + (PV ? 2 * DT : 0));
  constexpr int NDS = (QK ? DC : 0) + (PV ? 4 * DT : 0);
  if constexpr (NM > 0) {
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
    pipe_sched<0, NM, (NDS + NM - 1) / NM, 4, LD ? (NM / (2 * NI) > 0 ? NM / (2 * NI) : 1) : 0>();
  }
}

// Keys of half KH of a step at or past `real` get score -inf (probability 0): lane (l32, g) holds
// keys 32 KH + 8 (r / 4) + 4 g + r % 4 in S[r].
template <int KH, int QT>
__device__ __forceinline__ void pipe_mask(f32x16 (&s)[QT], int real, int g) {
  const int rr = real - 32 * KH - 4 * g;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[qt][r] = 8 * (r >> 2) + (r & 3) >= rr ? -INFINITY : s[qt][r];
  }
}

// A slot whose exponentials failed the sum check: each tile's m_i moves to the running max over its
// half-step s (every half-step the pipeline starts with holds a real key, so the max is finite;
// where it does not exceed m_i the factor is 1 and nothing changes), the output accumulators
// (which already include this slot's PV product) and l_i are rescaled, and the half's
// probabilities P[2 PH], P[2 PH + 1] and row sums are recomputed.
template <int D, int QT, int PH>
__device__ __forceinline__ void pipe_rescale(const f32x16 (&s)[QT], bf16x8 (&P)[4][QT], f32x16 (&oacc)[QT][D / 32],
                                             float (&m_i)[QT], float (&l_i)[QT], float (&rs)[QT], float scale_log2) {
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[qt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
    const float m_new = fmaxf(mx, m_i[qt]);
    const float alpha = __builtin_amdgcn_exp2f(m_i[qt] - m_new);
    l_i[qt] *= alpha;
    m_i[qt] = m_new;
#pragma unroll
    for (int t = 0; t < D / 32; ++t) oacc[qt][t] *= alpha;
    float r0 = 0.f, r1 = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(s[qt][r], scale_log2, -m_i[qt]));
      if (r & 1) r1 += pv;
      else r0 += pv;
      P[2 * PH + (r >> 3)][qt][r & 7] = (bf16_t)pv;
    }
    rs[qt] = r0 + r1;
  }
}

template <int QT>
__device__ __forceinline__ bool pipe_check(const float (&rs)[QT]) {
  bool bad = false;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) bad |= !(rs[qt] <= 65536.f);
  return __any(bad);
}

// Unit kernel. A workgroup of NW = BS / (32 QT) waves runs one unit; wave w owns the QT 32-query
// tiles vw = QT w .. QT w + QT - 1 (query rows [32 vw, 32 vw + 32) of the block). QT = 1: four
// waves (BS = 128), two workgroups per CU sharing its SIMDs; QT = 2: two waves of 64 queries with
// up to 512 registers each (one wave per SIMD), so every K / V fragment read feeds two products.
// KS = 2 (64-key blocks): each query tile gets two waves, one per 32-key half of every step, which
// share the K / V tiles and meet through LDS after the loop; a 64-query workgroup is then four
// waves, so its two workgroups per CU (the LDS ring allows two) give each SIMD two waves.
template <int D, int BS, int QT, int KS>
__global__ void __launch_bounds__(2 * BS / QT * KS) __attribute__((amdgpu_waves_per_eu(QT == 1 ? 2 : 1)))
bsa_unit_kernel(FwdParams p) {
  constexpr int NW = BS / (32 * QT);  // query waves
  constexpr int NWT = NW * KS;        // waves
  constexpr int NVW = NW * QT;        // 32-query tiles per workgroup
  constexpr int DC = D / 16, DT = D / 32;
  constexpr int TILE = 64 * D;  // elements of one K (or V) step tile
  // Two K and two V step tiles (64 KiB at D = 128: two workgroups per CU), one array per stage, fed
  // by direct-to-LDS loads; and each wave's step table (64 steps x (first row, real keys)).
  __shared__ __attribute__((aligned(1024))) bf16_t ks0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t ks1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t vs0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t vs1[TILE];
  __shared__ int steptab[NWT][64][2];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int qw = w % NW, kh = w / NW;  // query wave; key half (KS = 2)

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
  // Q^T fragments (B operand): lane holds Q[qi, 16c + 8g .. +8) of each of its tiles.
  int qi[QT];
  bool q_ok[QT];
  const bf16_t* qrow[QT];
  bf16x8 qf[QT][DC];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    qi[qt] = qb * BS + (qw * QT + qt) * 32 + l32;
    q_ok[qt] = qi[qt] < p.Lq;
    qrow[qt] = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)(q_ok[qt] ? qi[qt] : 0) * p.q_st;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      bf16x8 t = *(const bf16x8*)(qrow[qt] + c * 16 + g * 8);
      qf[qt][c] = q_ok[qt] ? t : bf16x8{};
    }
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

  // List entries one per lane, read once. A row of at most 64 visits is loaded whole and sorted by
  // block id, and split s of the row's ns units takes the sorted positions s, s + ns, s + 2 ns, ...:
  // every unit of a head (they run together on one XCD) then sweeps the whole key range in step
  // with the others, so the units that list a block fetch it at about the same time and share it in
  // L2. The visit order only changes the summation order. A longer row gives each unit one
  // contiguous slice of its list, sorted by block id the same way (a dense row is in order).
  const bool whole = n <= 64;
  const int lo = whole ? 0 : s_begin;
  const int take = whole ? n : s_end - s_begin;
  int my_j = 0;
  if (lane < take) my_j = p.index ? min(max(lo == 0 ? j0 : j1, 0), p.Nkv - 1) : lo + lane;
  if (whole || p.index) my_j = wave_sort_ascending(lane < take ? my_j : 0x7fffffff, lane);
  const bool mine = whole ? lane < n && lane % ns == split : lane < take;
  const int my_real = mine ? block_real(p, my_j, BS) : 0;

  // Step table: this unit's visits in processing order (the lanes with `mine`), each one 64-key
  // step or, for a block of more than 64 real keys, two. Lane s of tab_* describes step s: the byte
  // offsets of its first K and V rows in the head's slabs and its real key count (1..64). A unit
  // has at most 64 steps (split <= 32 visits of 128-key blocks, or 64 of 64-key blocks).
  const uint64_t vis = __ballot(mine && my_real > 0);
  const uint64_t two = BS == 128 ? __ballot(mine && my_real > 64) : 0ull;
  const int T = __popcll(vis) + __popcll(two);
  if ((vis >> lane) & 1) {
    const uint64_t below = (1ull << lane) - 1;
    const int first = __popcll(vis & below) + __popcll(two & below);
    steptab[w][first][0] = my_j * BS;
    steptab[w][first][1] = min(my_real, 64);
    if ((two >> lane) & 1) {
      steptab[w][first + 1][0] = my_j * BS + 64;
      steptab[w][first + 1][1] = my_real - 64;
    }
  }
  const int tab_row = lane < T ? steptab[w][lane][0] : 0;
  const int tab_real = lane < T ? steptab[w][lane][1] : 0;
  const int tab_koff = tab_row * (int)p.k_st * 2, tab_voff = tab_row * (int)p.v_st * 2;

  // Tile loads: this lane's loop-invariant chunk offsets; each tile gets a buffer descriptor that
  // starts at its first row and ends at the slab's end (rows past the slab read zeros), and a step
  // past the end of the table an empty one (zeros, no memory traffic).
  using NT = NextTile<D, NWT>;
  int k_off[NT::NI], v_off[NT::NI];
#pragma unroll
  for (int i = 0; i < NT::NI; ++i) {
    const int row = (i * NWT + w) * NT::RPI + lane / NT::CPR, pos = lane % NT::CPR;
    k_off[i] = (int)(row * p.k_st + (pos ^ k_swizzle<D>(row)) * 8) * 2;
    v_off[i] = (int)(row * p.v_st + (pos ^ v_swizzle(row)) * 8) * 2;
  }
  auto tile_rs = [&](int s, bool is_k) {
    const int off = __builtin_amdgcn_readlane(is_k ? tab_koff : tab_voff, s & 63);
    const bool ok = s < T;
    const char* base = (const char*)(is_k ? kbase : vbase) + (ok ? off : 0);
    const int bytes = ok ? (is_k ? p.k_slab_bytes : p.v_slab_bytes) - off : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, WA_BUF_DWORD3);
  };
  auto load_tile = [&](int s, bool is_k, bf16_t* lds) {
    const __amdgpu_buffer_rsrc_t rs = tile_rs(s, is_k);
#pragma unroll
    for (int i = 0; i < NT::NI; ++i) pipe_dma16(rs, lds + (i * NWT + w) * NT::RPI * D, is_k ? k_off[i] : v_off[i]);
  };
  // Q fragments in registers before the first tile loads (a later first use would wait for them)
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int c = 0; c < DC; ++c) asm volatile("" : "+v"(qf[qt][c]));
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

  f32x16 oacc[QT][DT];
  float m_i[QT], l_i[QT], neg_m[QT], rs[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[qt][t] = f32x16{};
    m_i[qt] = -INFINITY;
    l_i[qt] = 0.f;
  }
  auto set_neg_m = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) neg_m[qt] = -m_i[qt];
  };
  auto add_l = [&]() {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l_i[qt] += rs[qt];
  };

  // The pipeline. Step s's K tile lives in stage ks[s % 2] and its V tile in vs[s % 2]. Block b
  // (1 <= b < T) reads K(b) and V(b - 1) and loads K(b + 1) and V(b) into the stages the previous
  // block finished reading; its top waits for this wave's loads and then on the workgroup barrier,
  // so every wave's tiles of the block have landed and every wave is done with the stages being
  // refilled. Block 0 (QK of step 0) and block T (PV of step T - 1) are the pipeline's ends.
  // Exponentials run against the running max m_i, which may lag the scores: a slot is accepted
  // when every lane's sum of exponentials is at most 2^16 (so is each exponential: far from fp32 /
  // bf16 overflow). Otherwise (the first slot, or scores more than ~11 above m_i) m_i moves to the
  // half-step's max, the accumulators are rescaled and the half's exponentials recomputed; the
  // final normalization uses the same m_i, so the result does not depend on how far m_i lags.
  f32x16 S[2][QT];
  bf16x8 P[4][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    S[0][qt] = f32x16{};
    S[1][qt] = f32x16{};
#pragma unroll
    for (int c = 0; c < 4; ++c) P[c][qt] = bf16x8{};
  }
  const float sl2 = p.scale_log2;
  const PipeLoad no_load{};
  if constexpr (KS == 1) {
    if (T > 0) {
      load_tile(0, true, ks0);
      load_tile(1, true, ks1);
      load_tile(0, false, vs0);
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * NT::NI) : "memory");
      set_neg_m();
      pipe_slot<D, NWT, QT, 1, false, true, false, false>(S, P, oacc, qf, ks0, vs0, k_rd, v_rd, neg_m, sl2, no_load,
                                                         k_off, no_load, v_off, w, rs);
      int real_prev = __builtin_amdgcn_readlane(tab_real, 0);
      if (real_prev < 32) pipe_mask<0, QT>(S[0], real_prev, g);
      pipe_slot<D, NWT, QT, 0, true, true, false, false>(S, P, oacc, qf, ks0, vs0, k_rd, v_rd, neg_m, sl2, no_load,
                                                        k_off, no_load, v_off, w, rs);
      if (pipe_check<QT>(rs)) pipe_rescale<D, QT, 0>(S[0], P, oacc, m_i, l_i, rs, sl2);
      add_l();

      auto block = [&](auto par, int b) {
        constexpr int PAR = decltype(par)::value;
        bf16_t* const kcur = PAR ? ks1 : ks0;
        bf16_t* const knext = PAR ? ks0 : ks1;
        bf16_t* const vprev = PAR ? vs0 : vs1;
        bf16_t* const vcur = PAR ? vs1 : vs0;
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (real_prev < 64) pipe_mask<1, QT>(S[1], real_prev, g);
        const PipeLoad ldk{tile_rs(b + 1, true), knext}, ldv{tile_rs(b, false), vcur};
        set_neg_m();
        pipe_slot<D, NWT, QT, 1, true, true, true, true>(S, P, oacc, qf, kcur, vprev, k_rd, v_rd, neg_m, sl2, ldk, k_off,
                                                        ldv, v_off, w, rs);
        if (pipe_check<QT>(rs)) pipe_rescale<D, QT, 1>(S[1], P, oacc, m_i, l_i, rs, sl2);
        add_l();
        const int real = __builtin_amdgcn_readlane(tab_real, b);
        if (real < 32) pipe_mask<0, QT>(S[0], real, g);
        set_neg_m();
        pipe_slot<D, NWT, QT, 0, true, true, true, false>(S, P, oacc, qf, kcur, vprev, k_rd, v_rd, neg_m, sl2, no_load,
                                                         k_off, no_load, v_off, w, rs);
        if (pipe_check<QT>(rs)) pipe_rescale<D, QT, 0>(S[0], P, oacc, m_i, l_i, rs, sl2);
        add_l();
        real_prev = real;
      };
      int b = 1;
      for (; b + 1 < T; b += 2) {
        block(std::integral_constant<int, 1>{}, b);
        block(std::integral_constant<int, 0>{}, b + 1);
      }
      if (b < T) block(std::integral_constant<int, 1>{}, b);

      auto last = [&](auto par) {
        constexpr int PAR = decltype(par)::value;  // (T - 1) % 2: stage of V(T - 1)
        bf16_t* const vprev = PAR ? vs1 : vs0;
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if (real_prev < 64) pipe_mask<1, QT>(S[1], real_prev, g);
        set_neg_m();
        pipe_slot<D, NWT, QT, 1, true, false, true, false>(S, P, oacc, qf, ks0, vprev, k_rd, v_rd, neg_m, sl2, no_load,
                                                          k_off, no_load, v_off, w, rs);
        if (pipe_check<QT>(rs)) pipe_rescale<D, QT, 1>(S[1], P, oacc, m_i, l_i, rs, sl2);
        add_l();
        pipe_slot<D, NWT, QT, 0, false, false, true, false>(S, P, oacc, qf, ks0, vprev, k_rd, v_rd, neg_m, sl2, no_load,
                                                           k_off, no_load, v_off, w, rs);
      };
      if ((T - 1) & 1) last(std::integral_constant<int, 1>{});
      else last(std::integral_constant<int, 0>{});
    }
  } else {
    // Key split: this wave computes key half kh of every 64-key step, pipelined over steps with
    // one slot per step and K two steps ahead of V. Slot b (0 <= b < T) waits for K(b + 1) and
    // V(b - 1) (this wave's loads, then the workgroup barrier, after which every wave is done with
    // K(b) and V(b - 2)), loads K(b + 2) and V(b) into those stages, and runs the QK product of step
    // b + 1, the exponentials of step b (scores S[b % 2] -> P[2 (b % 2)], P[2 (b % 2) + 1]) and the
    // PV product of step b - 1 (the other P pair) as one interleaved slot; the sum check then
    // accepts step b's exponentials or rescales (the accumulators include step b - 1). Every slot
    // runs all three: a half without real keys is masked whole, so its exponentials are 0 — the
    // running max starts at -1e30 instead of -inf so that such a half, even as the wave's first,
    // rescales by exp2(0) = 1 rather than exp2(-inf + inf).
    auto run = [&](auto khc) {
      constexpr int KH = decltype(khc)::value;
      auto mask_step = [&](auto par, int b) {
        const int real = __builtin_amdgcn_readlane(tab_real, b & 63);
        if (real < 32 * (KH + 1)) pipe_mask<KH, QT>(S[decltype(par)::value], real, g);
        set_neg_m();
      };
      auto accept = [&](auto par) {
        if (pipe_check<QT>(rs)) pipe_rescale<D, QT, decltype(par)::value>(S[decltype(par)::value], P, oacc, m_i, l_i, rs, sl2);
        add_l();
      };
      auto slot = [&](auto par, int b) {
        constexpr int PAR = decltype(par)::value;  // b % 2
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        load_tile(b + 2, true, PAR ? ks1 : ks0);
        load_tile(b, false, PAR ? vs1 : vs0);
        mask_step(par, b);
        pipe_slot<D, NWT, QT, PAR, true, true, true, false, KH>(S, P, oacc, qf, PAR ? ks0 : ks1, PAR ? vs0 : vs1, k_rd,
                                                               v_rd, neg_m, sl2, no_load, k_off, no_load, v_off, w, rs);
        accept(par);
      };
      if (T > 0) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) m_i[qt] = -1e30f;
        load_tile(0, true, ks0);
        load_tile(1, true, ks1);
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NT::NI) : "memory");
        pipe_slot<D, NWT, QT, 1, false, true, false, false, KH>(S, P, oacc, qf, ks0, vs0, k_rd, v_rd, neg_m, sl2,
                                                               no_load, k_off, no_load, v_off, w, rs);
        // slot 0: no PV product yet
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        load_tile(2, true, ks0);
        load_tile(0, false, vs0);
        mask_step(std::integral_constant<int, 0>{}, 0);
        pipe_slot<D, NWT, QT, 0, true, true, false, false, KH>(S, P, oacc, qf, ks1, vs1, k_rd, v_rd, neg_m, sl2,
                                                              no_load, k_off, no_load, v_off, w, rs);
        accept(std::integral_constant<int, 0>{});
        int b = 1;
        for (; b + 1 < T; b += 2) {
          slot(std::integral_constant<int, 1>{}, b);
          slot(std::integral_constant<int, 0>{}, b + 1);
        }
        if (b < T) slot(std::integral_constant<int, 1>{}, b);
        // the last step's PV product (its V stage is vs[(T - 1) % 2], its P pair (T - 1) % 2)
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        if ((T - 1) & 1)
          pipe_slot<D, NWT, QT, 0, false, false, true, false, KH>(S, P, oacc, qf, ks0, vs1, k_rd, v_rd, neg_m, sl2,
                                                                 no_load, k_off, no_load, v_off, w, rs);
        else
          pipe_slot<D, NWT, QT, 1, false, false, true, false, KH>(S, P, oacc, qf, ks0, vs0, k_rd, v_rd, neg_m, sl2,
                                                                 no_load, k_off, no_load, v_off, w, rs);
      }
    };
    if (kh == 0) run(std::integral_constant<int, 0>{});
    else run(std::integral_constant<int, 1>{});
  }

  // every tile load has landed (block T waited for the last ones)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (KS == 2) {
    // The two key halves of each query tile meet: the half-1 wave leaves its running max, row sums
    // and accumulators in the drained ring, and the half-0 wave folds them into its own against the
    // larger max (lanes hold the same queries and key subsets in both waves).
    static_assert(QT * DT * 16 * 64 * 4 <= TILE * 2 && NW <= 2, "key-half exchange does not fit the ring");
    __syncthreads();  // every wave is done with the last step's tiles
    float* xo = (float*)(qw == 0 ? ks0 : ks1);
    float* xs = (float*)vs0 + qw * 2 * QT * 64;
    if (kh == 1) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
          for (int r = 0; r < 16; ++r) xo[((qt * DT + t) * 16 + r) * 64 + lane] = oacc[qt][t][r];
        }
        xs[(qt * 2) * 64 + lane] = m_i[qt];
        xs[(qt * 2 + 1) * 64 + lane] = l_i[qt];
      }
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const float m1 = xs[(qt * 2) * 64 + lane], l1 = xs[(qt * 2 + 1) * 64 + lane];
        const float mm = fmaxf(m_i[qt], m1);
        const float a0 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i[qt] - mm);
        const float a1 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
        l_i[qt] = l_i[qt] * a0 + l1 * a1;
        m_i[qt] = mm;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            oacc[qt][t][r] = oacc[qt][t][r] * a0 + xo[((qt * DT + t) * 16 + r) * 64 + lane] * a1;
        }
      }
    }
  }
  float inv[QT], lse2[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float lsum = l_i[qt] + __shfl_xor(l_i[qt], 32, 64);
    inv[qt] = lsum > 0.f ? 1.f / lsum : 0.f;
    // log2-sum-exp of this unit's keys; the row's natural-log lse is this times ln 2
    lse2[qt] = lsum > 0.f ? m_i[qt] + __log2f(lsum) : -INFINITY;
  }
  if (ns > 1) {
    // Normalized partial + log2-sum-exp; the row's last unit to arrive merges every partial, in
    // split order (its own is still in registers: the same fp32 values it stored). The row's units
    // may run on different XCDs, whose L2s are not coherent with each other, so the partials are
    // written and read with device-scope (sc1) buffer accesses instead of L2-wide write-back and
    // invalidate, and the arrival count is a device-scope atomic taken after this workgroup's
    // partial stores have completed; the last arrival loads the others' partials only after its
    // count has returned. A partial is stored in accumulator-fragment order (query tile, tile,
    // quad, lane), so every store and load instruction covers 1 KiB of contiguous memory.
    const int64_t slot0 = row * p.max_splits;
    constexpr int SLOT_BYTES = BS * D * 4;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(p.part_o + slot0 * (BS * D)), (short)0, ns * SLOT_BYTES, WA_BUF_DWORD3);
    auto frag_off = [&](int sp, int vw, int t, int rq) {
      return sp * SLOT_BYTES + (((vw * DT + t) * 4 + rq) * 64 + lane) * 16;
    };
    constexpr int SC1 = 16;  // cache policy: device-scope coherent
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      if (KS == 2 && kh == 1) break;  // the half-0 wave holds the merged tile
      const int vw = qw * QT + qt;
      if (g == 0)
        __hip_atomic_store(p.part_lse + (slot0 + split) * BS + vw * 32 + l32, lse2[qt], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 ov = {oacc[qt][t][rq * 4] * inv[qt], oacc[qt][t][rq * 4 + 1] * inv[qt],
                            oacc[qt][t][rq * 4 + 2] * inv[qt], oacc[qt][t][rq * 4 + 3] * inv[qt]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ov), prs, frag_off(split, vw, t, rq), 0, SC1);
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    int* s_last = &steptab[0][0][0];  // the step tables are no longer read
    if (tid == 0) {
      const bool last =
          __hip_atomic_fetch_add(p.arrivals + row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ns - 1;
      if (last) __hip_atomic_store(p.arrivals + row, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // reusable
      *s_last = last;
    }
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(*s_last)) return;  // uniform: one LDS word for every lane
    if (KS == 2 && kh == 1) return;
    // Another unit's partial comes in by direct-to-LDS loads into one free ring stage per query
    // tile (each wave reads back only what it loaded: no workgroup barrier), the first one together
    // with the first four log2-sum-exps, so a two-unit row merges after one round trip.
    static_assert(DT * 4 * 1024 <= TILE * 2 && NVW <= 4, "partial staging does not fit the ring stages");
    char* wbuf[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int vw = qw * QT + qt;
      wbuf[qt] = (char*)(vw == 0 ? ks0 : vw == 1 ? ks1 : vw == 2 ? vs0 : vs1);
    }
    auto fetch_part = [&](int sp) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq)
            lds_dma16_sc1(prs, wbuf[qt] + (t * 4 + rq) * 1024, frag_off(sp, qw * QT + qt, t, rq));
        }
      }
    };
    const int sp_first = split == 0 ? 1 : 0;
    fetch_part(sp_first);
    float lsv[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float* plse = p.part_lse + slot0 * BS + (qw * QT + qt) * 32 + l32;
#pragma unroll
      for (int sp = 0; sp < 4; ++sp)
        lsv[qt][sp] = sp >= ns ? -INFINITY
                               : sp == split ? lse2[qt]
                                             : __hip_atomic_load(plse + sp * BS, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    auto lse_of = [&](int qt, int sp) {
      if (sp < 4) return lsv[qt][sp];
      if (sp == split) return lse2[qt];
      return __hip_atomic_load(p.part_lse + slot0 * BS + (qw * QT + qt) * 32 + l32 + sp * BS, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    };
    float M[QT], Z[QT];
    f32x16 acc[QT][DT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      M[qt] = -INFINITY;
#pragma unroll 1
      for (int sp = 0; sp < ns; ++sp) M[qt] = fmaxf(M[qt], lse_of(qt, sp));
      Z[qt] = 0.f;
      if (M[qt] != -INFINITY) {
#pragma unroll 1
        for (int sp = 0; sp < ns; ++sp) {
          const float wgt = exp2f(lse_of(qt, sp) - M[qt]);
          if (wgt != 0.f) Z[qt] += wgt;
        }
      }
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[qt][t] = f32x16{};
    }
    // sum the weighted partials in split order (zero weights skipped)
#pragma unroll 1
    for (int sp = 0; sp < ns; ++sp) {
      if (sp == split) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float wgt = M[qt] != -INFINITY ? exp2f(lse_of(qt, sp) - M[qt]) : 0.f;
          if (wgt != 0.f) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
              for (int i = 0; i < 16; ++i) acc[qt][t][i] = fmaf(wgt, oacc[qt][t][i] * inv[qt], acc[qt][t][i]);
            }
          }
        }
        continue;
      }
      if (sp != sp_first) fetch_part(sp);  // the buffers are free: the previous partial was read
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const float wgt = M[qt] != -INFINITY ? exp2f(lse_of(qt, sp) - M[qt]) : 0.f;
        if (wgt != 0.f) {
#pragma unroll
          for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
              const f32x4 v = *(const f32x4*)(wbuf[qt] + (t * 4 + rq) * 1024 + lane * 16);
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[qt][t][rq * 4 + i] = fmaf(wgt, v[i], acc[qt][t][rq * 4 + i]);
            }
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next fetch
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int t = 0; t < DT; ++t) oacc[qt][t] = acc[qt][t];
      inv[qt] = Z[qt] > 0.f ? 1.f / Z[qt] : 0.f;
      lse2[qt] = Z[qt] > 0.f ? M[qt] + log2f(Z[qt]) : -INFINITY;
    }
  }
  if (KS == 2 && kh == 1) return;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    if (p.lse && g == 0 && q_ok[qt]) p.lse[((int64_t)b * p.H + h) * p.Lq + qi[qt]] = lse2[qt] * WA_LN2;
    write_output<D>(p, oacc[qt], inv[qt], qf[qt], qrow[qt], b, h, qi[qt], q_ok[qt], g, l32);
  }
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
int launch(const FwdParams& fp, int64_t rows, bool cleared, bool key_split, hipStream_t stream) {
  if (!cleared && fp.max_splits > 1) {  // (with one unit per row no unit counts arrivals)
    hipLaunchKernelGGL(bsa_clear_arrivals_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream,
                       fp.arrivals, rows);
    const int rc = wa_launch_status("bsa_fwd_clear");
    if (rc != WA_OK) return rc;
  }
  // 32 queries per wave. (64 per wave, QT = 2, halves the LDS reads per product but needs more
  // than 256 registers: as compiled today its loop moves ~1,600 values between AGPRs and VGPRs.)
  // 64-key blocks with long units split each step's keys between two waves (four waves per
  // workgroup: 712 against 735 us for the reference mode's sparse launch at the Wan shape, 180
  // visits per row); a short unit (the dense launch over ~9 compressed key blocks) does better
  // with its two waves' pipelined loop (57 against 62 us).
  constexpr int QT = 1;
  if constexpr (BS == 64) {
    if (key_split) {
      hipLaunchKernelGGL((bsa_unit_kernel<D, BS, QT, 2>), dim3(fp.n_units), dim3(4 * BS / QT), 0, stream, fp);
      return wa_launch_status("bsa_fwd_unit");
    }
  }
  hipLaunchKernelGGL((bsa_unit_kernel<D, BS, QT, 1>), dim3(fp.n_units), dim3(2 * BS / QT), 0, stream, fp);
  return wa_launch_status("bsa_fwd_unit");
}

// Workspace layout: the split partials (fp32 [rows * max_splits][BS][D] outputs, then
// [rows * max_splits][BS] log2-sum-exps; only when a row can take more than one unit), then the
// int32 arrival counters [rows], each region starting on a 256-byte boundary.
int64_t partial_bytes(int64_t rows, int64_t max_splits, int64_t block_size, int64_t D) {
  return max_splits > 1 ? (rows * max_splits * block_size * (D + 1) * 4 + 255) / 256 * 256 : 0;
}

// Default visits per unit: 16 for 128-key blocks (cfg 2: 8-32 listed blocks per row); 48 for
// 64-key blocks, whose Gini rows list ~180 blocks at the Wan shape (four units per row: the whole
// call 0.735 ms in graph replay against 0.755 at 64 visits, 0.755 at 40 and 0.85 at 32).
int64_t default_split(int64_t block_size) {
  return block_size == 64 ? WA_BSA_DEFAULT_SPLIT_64 : WA_BSA_DEFAULT_SPLIT;
}

int64_t max_splits_of(int64_t max_visits, int64_t split) {
  return max_visits > 0 ? (max_visits + split - 1) / split : 1;
}

int bsa_fwd_impl(const wa_bsa_fwd_args* a, void* workspace, void* stream);

}  // namespace

extern "C" int64_t wa_bsa_fwd_workspace_bytes(int64_t rows, int64_t max_visits, int64_t split, int64_t block_size,
                                              int64_t D) {
  if (split <= 0) split = default_split(block_size);
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
  const int64_t split = a->split_visits > 0 ? a->split_visits : default_split(a->block_size);
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
  const int64_t split = a->split_visits > 0 ? a->split_visits : default_split(a->block_size);
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
  // steps per unit: one per visit of a 64-key block
  const bool key_split = a->block_size == 64 && (split < max_visits ? split : max_visits) >= 32;
  if (a->D == 64 && a->block_size == 64) return launch<64, 64>(fp, rows, cleared, key_split, s);
  if (a->D == 64 && a->block_size == 128) return launch<64, 128>(fp, rows, cleared, false, s);
  if (a->D == 128 && a->block_size == 64) return launch<128, 64>(fp, rows, cleared, key_split, s);
  return launch<128, 128>(fp, rows, cleared, false, s);
}

}  // namespace
