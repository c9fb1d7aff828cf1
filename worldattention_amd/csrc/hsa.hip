// One call for the HSA forward of split heads (host code). It runs the same entry points, with the
// same arguments, as the Python orchestration of hsa_forward does for heads that take one branch
// each (top-k sparse heads, elu(x)+1 linear heads), from one workspace:
//  * the elu1 state pass and the gated readout of the linear heads, on the caller's side stream
//    when it passes one (forked from and joined back to its stream with the caller's two events),
//    else on its stream;
//  * block pooling of the sparse heads' queries and keys, top-k routing (which also clears the
//    sparse launch's arrival counters) and the block-sparse launch, on the caller's stream.
// With training outputs the linear heads' readout is kept unfused (lin) with its gate, and the
// sparse heads' log-sum-exp is written, which the one-call backward (wa_hsa_bwd) takes back:
//  * the sparse heads' gradients (wa_bsa_bwd) on the caller's stream;
//  * the gate backward (wa_hsa_fuse_bwd) and the elu1 backward (wa_elu1_bwd) of the linear heads
//    on the side stream; a bf16 dq of the linear heads is rounded from their fp32 sum at the end.
// An eager call then crosses from Python once instead of ~20 times (allocations, argument structs
// and launches). The calls keep no state between calls and take no lock: concurrent calls on
// different streams (each with its own side stream and events) are independent.
//
// Reference semantics: wan/modules/hsa/attention.py:153-259 (hsa_attention) with the north-star
// head modes, and its autograd (block_sparse_triton.py:353-368 for the sparse branch); each step
// follows the entry point it calls.
#include "common.h"

namespace {

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

struct HsaLayout {
  int64_t qp, kp, arrivals, thresholds, bsa, elu1, state, zsum, total;
};

HsaLayout hsa_layout(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D, int64_t bs, int64_t n_sparse,
                     int64_t n_linear, int64_t max_visits) {
  const int64_t nq = (Lq + bs - 1) / bs, nkv = (Lkv + bs - 1) / bs;
  const int64_t rows = B * n_sparse * nq;
  HsaLayout l{};
  int64_t o = 0;
  l.qp = o; o += align256(B * H * nq * D * 4);
  l.kp = o; o += align256(B * H * nkv * D * 4);
  l.arrivals = o; o += align256(rows * 4);
  l.thresholds = o; o += align256(H * 4);
  l.bsa = o; o += n_sparse > 0 ? align256(wa_bsa_fwd_workspace_bytes(rows, max_visits, 0, bs, D)) : 0;
  l.elu1 = o; o += n_linear > 0 ? align256(wa_elu1_state_workspace_bytes(B, n_linear, Lkv, D)) : 0;
  l.state = o; o += align256(B * n_linear * D * D * 4);
  l.zsum = o; o += align256(B * n_linear * D * 4);
  l.total = o;
  return l;
}

}  // namespace

extern "C" int64_t wa_hsa_fwd_workspace_bytes(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D,
                                              int64_t block_size, int64_t n_sparse, int64_t n_linear,
                                              int64_t max_visits) {
  if (block_size <= 0) return 0;
  return hsa_layout(B, H, Lq, Lkv, D, block_size, n_sparse, n_linear, max_visits).total;
}

namespace {
int hsa_branches(const wa_hsa_fwd_args* a, const HsaLayout& l, char* ws, void* stream, void* ls);

// Runs body(linear_stream) with the linear heads on the caller's side stream when `two`: fork
// (side waits for stream) before, join (stream waits for side) after, on every path once forked
// (a capture must end joined).
template <class F>
int with_side_stream(const char* who, bool two, void* stream, void* side_stream, void* fork_event, void* join_event,
                     F&& body) {
  hipStream_t side = (hipStream_t)side_stream;
  hipEvent_t fork = (hipEvent_t)fork_event, join = (hipEvent_t)join_event;
  if (two) {
    hipError_t e;
    if ((e = hipEventRecord(fork, (hipStream_t)stream)) != hipSuccess || (e = hipStreamWaitEvent(side, fork, 0)) != hipSuccess)
      return wa_fail((int)e, "%s: fork: %s", who, hipGetErrorString(e));
  }
  const int rc = body(two ? side_stream : stream);
  if (two) {
    hipError_t e;
    if ((e = hipEventRecord(join, side)) != hipSuccess || (e = hipStreamWaitEvent((hipStream_t)stream, join, 0)) != hipSuccess)
      return rc != WA_OK ? rc : wa_fail((int)e, "%s: join: %s", who, hipGetErrorString(e));
  }
  return rc;
}
}  // namespace

extern "C" int wa_hsa_fwd(const wa_hsa_fwd_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->k && a->v && a->o && a->workspace, "wa_hsa_fwd: null argument");
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_hsa_fwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0, "wa_hsa_fwd: bad sizes");
  WA_CHECK_ARG(a->n_sparse >= 0 && a->n_linear >= 0 && a->n_sparse + a->n_linear <= a->H,
               "wa_hsa_fwd: bad head counts");
  WA_CHECK_ARG(a->n_sparse == 0 || (a->sparse_heads && a->head_k && a->index && a->num && a->units),
               "wa_hsa_fwd: sparse heads need their list, per-head k, routing outputs and the unit table");
  WA_CHECK_ARG(a->n_linear == 0 || a->linear_heads, "wa_hsa_fwd: linear heads need their list");
  WA_CHECK_ARG(wa_aligned16(a->workspace), "wa_hsa_fwd: workspace must be 16-byte aligned");
  WA_CHECK_ARG(a->side_stream == nullptr || (a->fork_event && a->join_event),
               "wa_hsa_fwd: a side stream needs its fork and join events");
  WA_CHECK_ARG(a->lin == nullptr || (a->gate && a->lin_modes),
               "wa_hsa_fwd: an unfused linear output (lin) needs gate and lin_modes");
  WA_CHECK_ARG((a->state == nullptr) == (a->zsum == nullptr), "wa_hsa_fwd: state and zsum go together");
  if (a->B == 0 || a->Lq == 0) return WA_OK;
  const HsaLayout l =
      hsa_layout(a->B, a->H, a->Lq, a->Lkv, a->D, a->block_size, a->n_sparse, a->n_linear, a->max_visits);
  char* ws = (char*)a->workspace;
  const bool two = a->side_stream != nullptr && a->side_stream != stream && a->n_sparse > 0 && a->n_linear > 0;
  return with_side_stream("wa_hsa_fwd", two, stream, a->side_stream, a->fork_event, a->join_event,
                          [&](void* ls) { return hsa_branches(a, l, ws, stream, ls); });
}

namespace {

// The five launches; `ls` is the linear heads' stream (the caller's or the side stream).
int hsa_branches(const wa_hsa_fwd_args* a, const HsaLayout& l, char* ws, void* stream, void* ls) {
  const int64_t bs = a->block_size, D = a->D;
  const int64_t nq = (a->Lq + bs - 1) / bs, nkv = (a->Lkv + bs - 1) / bs;
  int rc = WA_OK;
  // Issue order: the sparse heads' chain first. A captured graph starts its branches in the
  // order they were captured, and the sparse chain (pool, route, attention) is the longer one.
  auto linear = [&]() -> int {
    if (a->n_linear > 0) {
      wa_elu1_state_args s{};
      s.k = a->k; s.k_sb = a->k_sb; s.k_st = a->k_st; s.k_sh = a->k_sh;
      s.v = a->v; s.v_sb = a->v_sb; s.v_st = a->v_st; s.v_sh = a->v_sh; s.dtype = WA_BF16;
      s.B = a->B; s.H = a->H; s.L = a->Lkv; s.D = D; s.heads = a->linear_heads; s.n_heads = a->n_linear;
      s.state = a->state ? a->state : (float*)(ws + l.state);
      s.zsum = a->zsum ? a->zsum : (float*)(ws + l.zsum);
      s.workspace = ws + l.elu1;
      if ((rc = wa_elu1_state(&s, ls)) != WA_OK) return rc;

      wa_elu1_readout_args o{};
      o.q = a->q; o.q_sb = a->q_sb; o.q_st = a->q_st; o.q_sh = a->q_sh; o.q_dtype = WA_BF16;
      o.state = s.state; o.zsum = s.zsum;
      o.B = a->B; o.H = a->H; o.L = a->Lq; o.D = D; o.heads = a->linear_heads; o.n_heads = a->n_linear;
      if (a->lin) {
        // training: the readout unfused into lin, then the gate (kept) and the gated output
        o.o = a->lin; o.o_sb = a->lin_sb; o.o_st = a->lin_st; o.o_sh = a->lin_sh; o.o_dtype = WA_F32;
        o.epilogue = WA_EPI_PLAIN;
        if ((rc = wa_elu1_readout(&o, ls)) != WA_OK) return rc;
        wa_hsa_fuse_args f{};
        f.q = a->q; f.q_sb = a->q_sb; f.q_st = a->q_st; f.q_sh = a->q_sh;
        f.lin = a->lin; f.l_sb = a->lin_sb; f.l_st = a->lin_st; f.l_sh = a->lin_sh;
        f.head_modes = a->lin_modes;
        f.out = a->o; f.o_sb = a->o_sb; f.o_st = a->o_st; f.o_sh = a->o_sh; f.o_dtype = a->o_dtype;
        f.gate = a->gate; f.g_sb = a->gate_sb; f.g_st = a->gate_st; f.g_sh = a->gate_sh;
        f.gate_w = a->gate_w; f.gate_b = a->gate_b;
        f.gate_pre_bf16 = a->gate_pre_bf16; f.gate_out_bf16 = a->gate_out_bf16;
        f.attn_round_bf16 = 1; f.lin_round_bf16 = a->lin_round_bf16;
        f.B = a->B; f.H = a->H; f.L = a->Lq; f.D = D;
        if ((rc = wa_hsa_fuse_fwd(&f, ls)) != WA_OK) return rc;
      } else {
        o.o = a->o; o.o_sb = a->o_sb; o.o_st = a->o_st; o.o_sh = a->o_sh; o.o_dtype = a->o_dtype;
        o.epilogue = WA_EPI_GATED; o.gate_w = a->gate_w; o.gate_b = a->gate_b;
        o.gate_pre_bf16 = a->gate_pre_bf16; o.gate_out_bf16 = a->gate_out_bf16; o.lin_round_bf16 = a->lin_round_bf16;
        if ((rc = wa_elu1_readout(&o, ls)) != WA_OK) return rc;
      }
    }
    return WA_OK;
  };
  auto sparse = [&]() -> int {
    if (a->n_sparse > 0) {
      // pooled queries and keys of the sparse heads (fp32 [B, H, blocks, D]; the reference's rounding)
      wa_pool_args pj[2] = {};
      const void* xs[2] = {a->q, a->k};
      const int64_t sb[2] = {a->q_sb, a->k_sb}, st[2] = {a->q_st, a->k_st}, sh[2] = {a->q_sh, a->k_sh};
      const int64_t len[2] = {a->Lq, a->Lkv}, nb[2] = {nq, nkv};
      const int64_t off[2] = {l.qp, l.kp};
      for (int i = 0; i < 2; ++i) {
        pj[i].x = xs[i]; pj[i].x_sb = sb[i]; pj[i].x_st = st[i]; pj[i].x_sh = sh[i]; pj[i].x_dtype = WA_BF16;
        pj[i].B = a->B; pj[i].L = len[i]; pj[i].H = a->H; pj[i].D = D; pj[i].block_size = bs; pj[i].num_blocks = nb[i];
        pj[i].heads = a->sparse_heads; pj[i].n_heads = a->n_sparse;
        pj[i].out = (float*)(ws + off[i]); pj[i].emulate_rounding = 1;
      }
      if ((rc = wa_block_mean_pool_n(pj, 2, stream)) != WA_OK) return rc;

      // top-k routing; it also zeroes the arrival counters of the sparse launch
      wa_route_args r{};
      r.q_pooled = (const float*)(ws + l.qp); r.k_pooled = (const float*)(ws + l.kp);
      r.B = a->B; r.H = a->H; r.Nq = nq; r.Nkv = nkv; r.D = D; r.mode = WA_ROUTE_TOPK;
      r.tau_min = 0.f; r.tau_span = 1.f; r.head_k = a->head_k;
      r.heads = a->sparse_heads; r.n_heads = a->n_sparse;
      r.index = a->index; r.num = a->num; r.thresholds = (float*)(ws + l.thresholds);
      r.clear = (int32_t*)(ws + l.arrivals); r.n_clear = a->B * a->n_sparse * nq;
      if ((rc = wa_route(&r, stream)) != WA_OK) return rc;

      // block-sparse attention of the sparse heads, rounded to bf16 (their output)
      wa_bsa_fwd_args f{};
      f.q = a->q; f.q_sb = a->q_sb; f.q_st = a->q_st; f.q_sh = a->q_sh;
      f.k = a->k; f.k_sb = a->k_sb; f.k_st = a->k_st; f.k_sh = a->k_sh;
      f.v = a->v; f.v_sb = a->v_sb; f.v_st = a->v_st; f.v_sh = a->v_sh;
      f.o = a->o; f.o_sb = a->o_sb; f.o_st = a->o_st; f.o_sh = a->o_sh; f.o_dtype = a->o_dtype;
      f.index = a->index; f.num = a->num; f.index_width = nkv;
      f.heads = a->sparse_heads; f.n_heads = a->n_sparse;
      f.B = a->B; f.H = a->H; f.Lq = a->Lq; f.Lkv = a->Lkv; f.D = D; f.block_size = bs;
      f.lse = a->lse;
      f.epilogue = WA_EPI_PLAIN; f.attn_round_bf16 = 1;
      f.workspace = ws + l.bsa; f.units = a->units; f.n_units = a->n_units; f.max_visits = a->max_visits;
      f.arrivals = (int32_t*)(ws + l.arrivals);
      if ((rc = wa_bsa_fwd(&f, stream)) != WA_OK) return rc;
    }
    return WA_OK;
  };
  if ((rc = sparse()) != WA_OK) return rc;
  return linear();
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------------
// wa_bsa_bwd with its dQ pass on a second stream (bsa_bwd.hip)
int wa_bsa_bwd_streams(const wa_bsa_bwd_args* a, void* stream, void* dq_stream, void* fork_event, void* join_event);

namespace {

struct HsaBwdLayout {
  int64_t dlin, dq32, bsa, elu1, fuse, total;
};

HsaBwdLayout hsa_bwd_layout(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D, int64_t bs, int64_t n_sparse,
                            int64_t n_linear) {
  HsaBwdLayout l{};
  int64_t o = 0;
  const int64_t blhd = n_linear > 0 ? align256(B * Lq * H * D * 4) : 0;  // fp32 [B, Lq, H, D]
  l.dlin = o; o += blhd;
  l.dq32 = o; o += blhd;  // the linear heads' fp32 dq when dq is bf16
  l.bsa = o; o += n_sparse > 0 ? align256(wa_bsa_bwd_workspace_bytes(B, n_sparse, Lq, Lkv, D, bs)) : 0;
  l.elu1 = o; o += n_linear > 0 ? align256(wa_elu1_bwd_workspace_bytes(B, n_linear, Lq, D)) : 0;
  l.fuse = o; o += n_linear > 0 ? align256(wa_hsa_fuse_bwd_workspace_bytes(B, H, Lq, D)) : 0;
  l.total = o;
  return l;
}

// fp32 -> bf16 (round to nearest even) of the listed heads of a BLHD tensor, 8 channels a thread
__global__ void __launch_bounds__(256) round_heads_kernel(const float* __restrict__ src, int64_t s_sb, int64_t s_st,
                                                          int64_t s_sh, bf16_t* __restrict__ dst, int64_t d_sb,
                                                          int64_t d_st, int64_t d_sh, const int32_t* heads,
                                                          int n_heads, int L, int D, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int per_row = D / 8;
  const int c8 = (int)(i % per_row);
  const int64_t r = i / per_row;
  const int t = (int)(r % L);
  const int64_t bh = r / L;
  const int h = heads[bh % n_heads], b = (int)(bh / n_heads);
  const float4* s = (const float4*)(src + b * s_sb + (int64_t)t * s_st + h * s_sh + 8 * c8);
  const float4 x0 = s[0], x1 = s[1];
  bf16x8 y;
  y[0] = (bf16_t)x0.x; y[1] = (bf16_t)x0.y; y[2] = (bf16_t)x0.z; y[3] = (bf16_t)x0.w;
  y[4] = (bf16_t)x1.x; y[5] = (bf16_t)x1.y; y[6] = (bf16_t)x1.z; y[7] = (bf16_t)x1.w;
  *(bf16x8*)(dst + b * d_sb + (int64_t)t * d_st + h * d_sh + 8 * c8) = y;
}

int hsa_bwd_sparse(const wa_hsa_bwd_args* a, const HsaBwdLayout& l, char* ws, void* stream) {
  const bool dq_side = a->dq_stream && a->dq_stream != stream;
  const int64_t bs = a->block_size;
  wa_bsa_bwd_args g{};
  g.q = a->q; g.q_sb = a->q_sb; g.q_st = a->q_st; g.q_sh = a->q_sh;
  g.k = a->k; g.k_sb = a->k_sb; g.k_st = a->k_st; g.k_sh = a->k_sh;
  g.v = a->v; g.v_sb = a->v_sb; g.v_st = a->v_st; g.v_sh = a->v_sh;
  g.o = a->o; g.o_sb = a->o_sb; g.o_st = a->o_st; g.o_sh = a->o_sh; g.o_dtype = a->o_dtype;
  g.dout = a->dout; g.d_sb = a->d_sb; g.d_st = a->d_st; g.d_sh = a->d_sh; g.dout_dtype = a->dout_dtype;
  g.lse = a->lse; g.index = a->index; g.num = a->num; g.index_width = (a->Lkv + bs - 1) / bs;
  g.heads = a->sparse_heads; g.n_heads = a->n_sparse;
  g.B = a->B; g.H = a->H; g.Lq = a->Lq; g.Lkv = a->Lkv; g.D = a->D; g.block_size = bs;
  g.dq = (float*)a->dq; g.dq_sb = a->dq_sb; g.dq_st = a->dq_st; g.dq_sh = a->dq_sh; g.dq_dtype = a->dq_dtype;
  g.dk = a->dk; g.dk_sb = a->dk_sb; g.dk_st = a->dk_st; g.dk_sh = a->dk_sh;
  g.dv = a->dv; g.dv_sb = a->dv_sb; g.dv_st = a->dv_st; g.dv_sh = a->dv_sh; g.dkv_dtype = a->dkv_dtype;
  g.workspace = ws + l.bsa;
  return wa_bsa_bwd_streams(&g, stream, dq_side ? a->dq_stream : nullptr, a->dq_fork_event, a->dq_join_event);
}

int hsa_bwd_linear(const wa_hsa_bwd_args* a, const HsaBwdLayout& l, char* ws, void* ls) {
  const int64_t H = a->H, D = a->D;
  // contiguous fp32 BLHD scratch: dlin, and dq when the caller's dq is bf16
  const int64_t c_sb = a->Lq * H * D, c_st = H * D, c_sh = D;
  float* dlin = (float*)(ws + l.dlin);
  const bool dq32 = a->dq_dtype == WA_F32;
  float* dq = dq32 ? (float*)a->dq : (float*)(ws + l.dq32);
  const int64_t dq_sb = dq32 ? a->dq_sb : c_sb, dq_st = dq32 ? a->dq_st : c_st, dq_sh = dq32 ? a->dq_sh : c_sh;

  wa_hsa_fuse_args f{};
  f.q = a->q; f.q_sb = a->q_sb; f.q_st = a->q_st; f.q_sh = a->q_sh;
  f.lin = a->lin; f.l_sb = a->lin_sb; f.l_st = a->lin_st; f.l_sh = a->lin_sh;
  f.head_modes = a->lin_modes;
  f.gate = (float*)a->gate; f.g_sb = a->gate_sb; f.g_st = a->gate_st; f.g_sh = a->gate_sh;
  f.gate_w = a->gate_w; f.gate_b = a->gate_b;
  f.gate_pre_bf16 = a->gate_pre_bf16; f.gate_out_bf16 = a->gate_out_bf16;
  f.attn_round_bf16 = 0; f.lin_round_bf16 = a->lin_round_bf16;
  f.dout = a->dout; f.d_sb = a->d_sb; f.d_st = a->d_st; f.d_sh = a->d_sh; f.dout_dtype = a->dout_dtype;
  f.dlin = dlin; f.dl_sb = c_sb; f.dl_st = c_st; f.dl_sh = c_sh;
  f.dq = dq; f.dq_sb = dq_sb; f.dq_st = dq_st; f.dq_sh = dq_sh; f.dq_accumulate = 0;
  f.dgate_w = a->dgate_w; f.dgate_b = a->dgate_b; f.workspace = ws + l.fuse;
  f.B = a->B; f.H = H; f.L = a->Lq; f.D = D;
  int rc = wa_hsa_fuse_bwd(&f, ls);
  if (rc != WA_OK) return rc;

  wa_elu1_bwd_args e{};
  e.q = a->q; e.q_sb = a->q_sb; e.q_st = a->q_st; e.q_sh = a->q_sh; e.q_dtype = WA_BF16;
  e.k = a->k; e.k_sb = a->k_sb; e.k_st = a->k_st; e.k_sh = a->k_sh;
  e.v = a->v; e.v_sb = a->v_sb; e.v_st = a->v_st; e.v_sh = a->v_sh; e.kv_dtype = WA_BF16;
  e.dout = dlin; e.d_sb = c_sb; e.d_st = c_st; e.d_sh = c_sh; e.dout_dtype = WA_F32;
  e.state = a->state; e.zsum = a->zsum;
  e.dq = dq; e.dq_sb = dq_sb; e.dq_st = dq_st; e.dq_sh = dq_sh; e.dq_accumulate = 1;
  e.dk = a->dk; e.dk_sb = a->dk_sb; e.dk_st = a->dk_st; e.dk_sh = a->dk_sh; e.dk_accumulate = 0;
  e.dv = a->dv; e.dv_sb = a->dv_sb; e.dv_st = a->dv_st; e.dv_sh = a->dv_sh; e.dv_accumulate = 0;
  e.heads = a->linear_heads; e.n_heads = a->n_linear;
  e.B = a->B; e.H = H; e.Lq = a->Lq; e.Lkv = a->Lkv; e.D = D;
  e.workspace = ws + l.elu1; e.dkv_dtype = a->dkv_dtype;
  if ((rc = wa_elu1_bwd(&e, ls)) != WA_OK) return rc;

  if (!dq32) {
    const int64_t total = a->B * a->n_linear * a->Lq * (D / 8);
    hipLaunchKernelGGL(round_heads_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)ls, dq,
                       c_sb, c_st, c_sh, (bf16_t*)a->dq, a->dq_sb, a->dq_st, a->dq_sh, a->linear_heads,
                       (int)a->n_linear, (int)a->Lq, (int)D, total);
    return wa_launch_status("hsa_bwd_round_dq");
  }
  return WA_OK;
}

}  // namespace

extern "C" int64_t wa_hsa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D,
                                              int64_t block_size, int64_t n_sparse, int64_t n_linear) {
  if (block_size <= 0) return 0;
  return hsa_bwd_layout(B, H, Lq, Lkv, D, block_size, n_sparse, n_linear).total;
}

extern "C" int wa_hsa_bwd(const wa_hsa_bwd_args* a, void* stream) {
  WA_CHECK_ARG(a && a->q && a->k && a->v && a->dout && a->dq && a->dk && a->dv && a->workspace,
               "wa_hsa_bwd: null argument");
  WA_CHECK_ARG(a->block_size == 64 || a->block_size == 128, "wa_hsa_bwd: block size %lld not in {64, 128}",
               (long long)a->block_size);
  WA_CHECK_ARG(a->D == 64 || a->D == 128, "wa_hsa_bwd: head dim %lld not in {64, 128}", (long long)a->D);
  WA_CHECK_ARG(a->B >= 0 && a->H > 0 && a->Lq >= 0 && a->Lkv > 0, "wa_hsa_bwd: bad sizes");
  WA_CHECK_ARG(a->n_sparse >= 0 && a->n_linear >= 0 && a->n_sparse + a->n_linear <= a->H,
               "wa_hsa_bwd: bad head counts");
  WA_CHECK_ARG(a->n_sparse == 0 || (a->sparse_heads && a->index && a->num && a->lse && a->o),
               "wa_hsa_bwd: sparse heads need their list, routing, lse and output");
  WA_CHECK_ARG(a->n_linear == 0 || (a->linear_heads && a->lin_modes && a->lin && a->gate && a->state && a->zsum),
               "wa_hsa_bwd: linear heads need their list, modes, lin, gate, state and zsum");
  WA_CHECK_ARG(a->gate_w == nullptr || (a->dgate_w && a->dgate_b), "wa_hsa_bwd: gate_w needs dgate_w and dgate_b");
  WA_CHECK_ARG(a->dq_dtype == WA_F32 || a->dq_dtype == WA_BF16, "wa_hsa_bwd: bad dq dtype");
  WA_CHECK_ARG(a->dkv_dtype == WA_F32 || a->dkv_dtype == WA_BF16, "wa_hsa_bwd: bad dk / dv dtype");
  WA_CHECK_ARG(a->dq_dtype == WA_F32 || (wa_aligned16(a->dq) && a->dq_sb % 8 == 0 && a->dq_st % 8 == 0 &&
                                         a->dq_sh % 8 == 0),
               "wa_hsa_bwd: a bf16 dq must be 16-byte aligned with strides in multiples of 8 elements");
  WA_CHECK_ARG(wa_aligned16(a->workspace), "wa_hsa_bwd: workspace must be 16-byte aligned");
  WA_CHECK_ARG(a->side_stream == nullptr || (a->fork_event && a->join_event),
               "wa_hsa_bwd: a side stream needs its fork and join events");
  WA_CHECK_ARG(a->dq_stream == nullptr || (a->dq_fork_event && a->dq_join_event),
               "wa_hsa_bwd: a dQ stream needs its fork and join events");
  if (a->B == 0 || a->Lq == 0) return WA_OK;
  const HsaBwdLayout l = hsa_bwd_layout(a->B, a->H, a->Lq, a->Lkv, a->D, a->block_size, a->n_sparse, a->n_linear);
  char* ws = (char*)a->workspace;
  const bool two = a->side_stream != nullptr && a->side_stream != stream && a->n_sparse > 0 && a->n_linear > 0;
  return with_side_stream("wa_hsa_bwd", two, stream, a->side_stream, a->fork_event, a->join_event, [&](void* ls) {
    // the linear heads are issued first (their side stream starts while the sparse launches queue)
    int rc = a->n_linear > 0 ? hsa_bwd_linear(a, l, ws, ls) : WA_OK;
    if (rc == WA_OK && a->n_sparse > 0) rc = hsa_bwd_sparse(a, l, ws, stream);
    return rc;
  });
}
