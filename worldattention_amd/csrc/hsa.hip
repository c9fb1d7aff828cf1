// One call for the HSA forward of split heads (host code). It runs the same entry points, with the
// same arguments, as the Python orchestration of hsa_forward does for heads that take one branch
// each (top-k sparse heads, elu(x)+1 linear heads), from one workspace:
//  * the elu1 state pass and the gated readout of the linear heads, on the caller's side stream
//    when it passes one (forked from and joined back to its stream with the caller's two events),
//    else on its stream;
//  * block pooling of the sparse heads' queries and keys, top-k routing (which also clears the
//    sparse launch's arrival counters) and the block-sparse launch, on the caller's stream.
// An eager call then crosses from Python once instead of ~20 times (allocations, argument structs
// and launches). The call keeps no state between calls and takes no lock: concurrent calls on
// different streams (each with its own side stream and events) are independent.
//
// Reference semantics: wan/modules/hsa/attention.py:153-259 (hsa_attention) with the north-star
// head modes; each step follows the entry point it calls.
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
  if (a->B == 0 || a->Lq == 0) return WA_OK;
  const HsaLayout l =
      hsa_layout(a->B, a->H, a->Lq, a->Lkv, a->D, a->block_size, a->n_sparse, a->n_linear, a->max_visits);
  char* ws = (char*)a->workspace;
  const bool two = a->side_stream != nullptr && a->side_stream != stream && a->n_sparse > 0 && a->n_linear > 0;
  hipStream_t side = (hipStream_t)a->side_stream;
  hipEvent_t fork = (hipEvent_t)a->fork_event, join = (hipEvent_t)a->join_event;
  if (two) {
    hipError_t e;
    if ((e = hipEventRecord(fork, (hipStream_t)stream)) != hipSuccess || (e = hipStreamWaitEvent(side, fork, 0)) != hipSuccess)
      return wa_fail((int)e, "wa_hsa_fwd: fork: %s", hipGetErrorString(e));
  }
  int rc = hsa_branches(a, l, ws, stream, two ? (void*)side : stream);
  // the caller's stream joins the side stream on every path once forked (a capture must end joined)
  if (two) {
    hipError_t e;
    if ((e = hipEventRecord(join, side)) != hipSuccess || (e = hipStreamWaitEvent((hipStream_t)stream, join, 0)) != hipSuccess)
      return rc != WA_OK ? rc : wa_fail((int)e, "wa_hsa_fwd: join: %s", hipGetErrorString(e));
  }
  return rc;
}

namespace {

// The five launches; `ls` is the linear heads' stream (the caller's or the side stream).
int hsa_branches(const wa_hsa_fwd_args* a, const HsaLayout& l, char* ws, void* stream, void* ls) {
  const int64_t bs = a->block_size, D = a->D;
  const int64_t nq = (a->Lq + bs - 1) / bs, nkv = (a->Lkv + bs - 1) / bs;
  int rc = WA_OK;
  // the linear heads are issued first, as in the Python orchestration
  if (a->n_linear > 0) {
    wa_elu1_state_args s{};
    s.k = a->k; s.k_sb = a->k_sb; s.k_st = a->k_st; s.k_sh = a->k_sh;
    s.v = a->v; s.v_sb = a->v_sb; s.v_st = a->v_st; s.v_sh = a->v_sh; s.dtype = WA_BF16;
    s.B = a->B; s.H = a->H; s.L = a->Lkv; s.D = D; s.heads = a->linear_heads; s.n_heads = a->n_linear;
    s.state = (float*)(ws + l.state); s.zsum = (float*)(ws + l.zsum); s.workspace = ws + l.elu1;
    if ((rc = wa_elu1_state(&s, ls)) != WA_OK) return rc;

    wa_elu1_readout_args o{};
    o.q = a->q; o.q_sb = a->q_sb; o.q_st = a->q_st; o.q_sh = a->q_sh; o.q_dtype = WA_BF16;
    o.state = s.state; o.zsum = s.zsum;
    o.o = a->o; o.o_sb = a->o_sb; o.o_st = a->o_st; o.o_sh = a->o_sh; o.o_dtype = a->o_dtype;
    o.B = a->B; o.H = a->H; o.L = a->Lq; o.D = D; o.heads = a->linear_heads; o.n_heads = a->n_linear;
    o.epilogue = WA_EPI_GATED; o.gate_w = a->gate_w; o.gate_b = a->gate_b;
    o.gate_pre_bf16 = a->gate_pre_bf16; o.gate_out_bf16 = a->gate_out_bf16; o.lin_round_bf16 = a->lin_round_bf16;
    if ((rc = wa_elu1_readout(&o, ls)) != WA_OK) return rc;
  }

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
    f.epilogue = WA_EPI_PLAIN; f.attn_round_bf16 = 1;
    f.workspace = ws + l.bsa; f.units = a->units; f.n_units = a->n_units; f.max_visits = a->max_visits;
    f.arrivals = (int32_t*)(ws + l.arrivals);
    if ((rc = wa_bsa_fwd(&f, stream)) != WA_OK) return rc;
  }
  return WA_OK;
}

}  // namespace
