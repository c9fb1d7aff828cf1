/*
 * worldattention_amd — C ABI of the MI355X (gfx950) HSA + HKV attention path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, launches on the
 * caller's HIP stream (`stream` is a hipStream_t passed as void*), allocates nothing and keeps no
 * global device state, except wa_bsa_fwd_noalloc, whose workspace is a static device array of the
 * library. Inputs, outputs, workspaces, side streams and events are owned by the caller; workspace
 * sizes come from the matching *_workspace_bytes query.
 *
 * Return value: WA_OK (0) on success; a negative WA_ERR_* for argument errors; a positive
 * hipError_t for runtime failures. wa_last_error() returns the calling thread's last message.
 *
 * Tensor convention ("BLHD"): element (b, t, h, c) of a [B, L, H, C] tensor lives at
 * ptr + b*sb + t*st + h*sh + c, with strides in elements and the channel dim contiguous — the
 * layout of the reference's q/k/v and KV-cache slices, so no transposes or pad copies are needed.
 *
 * Reference: alibaba-damo-academy/WorldAttention (paths relative to its repository root).
 */
#ifndef WORLDATTENTION_AMD_H
#define WORLDATTENTION_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WA_OK 0
#define WA_ERR_ARG (-1)
#define WA_ERR_UNSUPPORTED (-2)
#define WA_ERR_IO (-3)

enum { WA_F32 = 0, WA_BF16 = 1 };
enum { WA_ROUTE_GINI = 0, WA_ROUTE_TOPK = 1 };
enum { WA_EPI_PLAIN = 0, WA_EPI_FUSE = 1, WA_EPI_GATED = 2 };

/* Library version (major*10000 + minor*100 + patch) and the last error message of this thread. */
int wa_version(void);
const char* wa_last_error(void);

/* ------------------------------------------------------------------------------------------ */
/* Routing                                                                                     */
/* ------------------------------------------------------------------------------------------ */

/* Block mean pooling of a BLHD tensor into [B, H, num_blocks, D] fp32.
 * Replaces block_mean_pool, wan/modules/hsa/routing.py:45-61 (called at attention.py:214-215).
 * The last block may be partial (L < num_blocks*block_size); it averages its real tokens only.
 * With emulate_rounding set, the reference's rounding is reproduced for a bf16 input: a
 * block-aligned L gives bf16(sum/block_size); otherwise fp32(bf16(sum)) / real_count.
 * Only the heads listed in `heads` (device int32[n_heads]; NULL = all) are written. */
typedef struct wa_pool_args {
  const void* x; int64_t x_sb, x_st, x_sh; int32_t x_dtype;
  int64_t B, L, H, D, block_size, num_blocks;
  const int32_t* heads; int64_t n_heads;
  float* out;
  int32_t emulate_rounding;
  /* Block range and sums (no reference counterpart; the cache-write side of causal_model.py:286-327
   * keeps them): blocks first_block .. first_block + num_blocks - 1 are written (L still counts
   * tokens from token 0 of x), into an output of out_blocks blocks (0: first_block + num_blocks);
   * with store_sums the fp32 block sums (in the order the means are formed from) are written
   * instead of the means. */
  int64_t first_block, out_blocks;
  int32_t store_sums;
} wa_pool_args;
int wa_block_mean_pool(const wa_pool_args* args, void* stream);
/* Several pooling jobs (e.g. the query and key tensors of one routing call) with as few launches
 * as possible: jobs of one kernel variant (dtype, 16-byte alignment) share a launch. No reference
 * counterpart: the reference pools q and k with two calls (routing.py:45-61, attention.py:212-213). */
int wa_block_mean_pool_n(const wa_pool_args* jobs, int32_t n_jobs, void* stream);

/* Block routing for one call: the block attention map softmax(qp kp^T / sqrt(D)) (or a given
 * map), the stable descending permutation of every row, and the selected count per row.
 * Replaces block_attention_map + build_block_routing, wan/modules/hsa/routing.py:64-118
 * (called at attention.py:212-222), and adds the north-star per-head top-k rule.
 *   GINI: thresholds[h] = tau_min + mean_{b,i} gini[b,h,i] * tau_span; num counts the sorted
 *         slots whose exclusive prefix (fp32 of a sequential double cumsum, minus the slot) is
 *         below the threshold — the reference's rounding points (routing.py:95-113).
 *   TOPK: num = min(head_k[h], Nkv).
 * index: [B, H, Nq, Nkv] int32, descending by weight, ties lowest block id first.
 * num:   [B, H, Nq] int32. mask (optional): [B, H, Nq, Nkv] uint8 selection mask.
 * probs (optional input) replaces the q_pooled/k_pooled map computation; probs_out (optional)
 * receives the computed map. For heads not listed in `heads`, num rows are written 0 and index /
 * mask rows are not written; thresholds (optional with TOPK) is written for every head, 0 where no
 * Gini threshold applies. No output needs initializing.
 * clear (optional, no reference counterpart): n_clear int32 words the launch sets to 0 — the
 * arrivals buffer of the wa_bsa_fwd launch that follows, cleared here without a launch of its own. */
typedef struct wa_route_args {
  const float* probs;
  const float* q_pooled;
  const float* k_pooled;
  int64_t B, H, Nq, Nkv, D;
  int32_t mode;
  float tau_min, tau_span;
  const int32_t* head_k;
  const int32_t* heads; int64_t n_heads;
  int32_t* index;
  int32_t* num;
  float* thresholds;
  uint8_t* mask;
  float* probs_out;
  void* workspace;
  int32_t* clear; int64_t n_clear;
  /* k_sum_len > 0 (no reference counterpart): k_pooled holds the fp32 block sums that
   * wa_block_mean_pool writes with store_sums for a key tensor of k_sum_len tokens in blocks of
   * block_size (k_sum_bf16: the keys are bf16); the launch forms from them exactly the block means
   * a pooling of those keys gives (routing.py:45-61 rounding), so the keys need no pooling pass.
   * k_pooled_blocks: blocks per (batch, head) row of k_pooled (0: Nkv), so the sums of a cache
   * longer than the routed keys are read in place. */
  int64_t k_sum_len, block_size;
  int32_t k_sum_bf16;
  int64_t k_pooled_blocks;
  /* scale (0: D^-1/2): the logit scale of the map. A caller that pads the head dim passes the
   * scale of its original head dim (routing.py:66 scales by the pooled vectors' own length). */
  float scale;
} wa_route_args;
int64_t wa_route_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nkv);
int wa_route(const wa_route_args* args, void* stream);

/* Appends new tokens to a KV cache and keeps its key block sums current. Replaces the cache write
 * of causal_model.py:286-327 (kv_cache["k"/"v"][:, start:end] = roped k / v): new_k / new_v
 * [B, n, H, D] (BLHD strides, bf16 or fp32 like the cache) are copied to cache tokens
 * [start, start + n) of cache_k / cache_v [B, cap, H, D]. With k_sums (optional, fp32
 * [B, H, ceil(cap / block_size), D], no reference counterpart), the sums of every key block that
 * holds a new token are recomputed over the cache tokens [0, start + n) (wa_block_mean_pool's
 * store_sums, same order), for the heads listed in `heads` (NULL = all): a later routing call over
 * the first start + n tokens reads them instead of pooling the keys (wa_route's k_sum_len). */
typedef struct wa_kv_append_args {
  void* cache_k; int64_t ck_sb, ck_st, ck_sh;
  void* cache_v; int64_t cv_sb, cv_st, cv_sh;
  const void* new_k; int64_t nk_sb, nk_st, nk_sh;
  const void* new_v; int64_t nv_sb, nv_st, nv_sh;
  int32_t dtype;
  int64_t B, cap, H, D, start, n;
  float* k_sums; int64_t block_size;
  const int32_t* heads; int64_t n_heads;
} wa_kv_append_args;
int wa_kv_append(const wa_kv_append_args* args, void* stream);

/* QKV epilogue of one cached causal attention step (after the q / k / v projections). Replaces
 * norm_q / norm_k (WanRMSNorm, wan/modules/model.py:70-86, applied at causal_model.py:166-169),
 * causal_rope_apply of q and k (causal_model.py:34-62, called at :275-281) and the cache write of
 * the roped keys and the values (causal_model.py:358-365 / :393-400, committed at :1089-1113):
 *   q_out[b, s]              = rope(norm_q(q[b, s]))            s < n
 *   cache_k[b, ws + t]       = rope(norm_k(k[b, so + t]))       t < write_len
 *   cache_v[b, ws + t]       = v[b, so + t]
 * (ws = write_start, so = src_offset). q, k, v, q_out and the caches are [B, *, H, D] BLHD of one
 * dtype (bf16 or fp32). rope: the 3-D RoPE of token s's position (frame start_frame + s / (gh*gw),
 * row, column) in the grid_f x grid_h x grid_w grid, from `freqs` = the model's complex128 table
 * [f_rows, D / 2] as fp64 (re, im) pairs; products in fp64, rounded to fp32, then to the dtype.
 * Tokens s >= grid_f * grid_h * grid_w pass through unrotated. norm (q_norm_w and k_norm_w [H * D],
 * w_dtype bf16 or fp32; both NULL: no norm): x * rsqrt(mean(x^2) + eps) over a token's H * D
 * channels in fp32, summed in torch's CPU order, rounded to the dtype, times the weight in the wider
 * of the two dtypes. With k_sums (fp32 [B, H, ceil(cap / block_size), D], no reference
 * counterpart) the key block sums of the written blocks are then refreshed as wa_kv_append does.
 * sample_grids (optional, HOST int64 [B][3]): each sample's own (f, h, w), as the reference's
 * per-sample loop over grid_sizes (causal_model.py:43) takes them; grid_f / grid_h / grid_w are then
 * ignored. Samples whose grids differ run in separate launches. */
typedef struct wa_qkv_epilogue_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  int32_t dtype;
  int64_t B, n, H, D;
  void* q_out; int64_t qo_sb, qo_st, qo_sh;
  void* cache_k; int64_t ck_sb, ck_st, ck_sh;
  void* cache_v; int64_t cv_sb, cv_st, cv_sh;
  int64_t cap, write_start, src_offset, write_len;
  const double* freqs; int64_t f_rows;
  int64_t grid_f, grid_h, grid_w, start_frame;
  const void* q_norm_w; const void* k_norm_w; int32_t w_dtype; float eps;
  float* k_sums; int64_t block_size;
  const int64_t* sample_grids;
} wa_qkv_epilogue_args;
int wa_qkv_epilogue(const wa_qkv_epilogue_args* args, void* stream);

/* Sliding-window roll of a KV cache, in place. Replaces the clone-and-shift of
 * causal_model.py:326-356 (and its commit, :1034-1087): tokens [sink + evicted,
 * sink + evicted + rolled) of cache_k / cache_v move to [sink, sink + rolled); with k_coarse /
 * v_coarse (same dtype, [B, coarse_cap, H, D]) coarse rows [c_src, c_src + c_rows) move to
 * [c_dst, c_dst + c_rows). No copy of the cache is made: the move runs in launches of at most
 * `evicted` tokens, each of which overwrites only tokens earlier launches have read. With k_sums,
 * the key block sums over [sink, sink + rolled) are recomputed (heads as in wa_kv_append). */
typedef struct wa_kv_roll_args {
  void* cache_k; int64_t ck_sb, ck_st, ck_sh;
  void* cache_v; int64_t cv_sb, cv_st, cv_sh;
  int32_t dtype;
  int64_t B, cap, H, D;
  int64_t sink, evicted, rolled;
  float* k_sums; int64_t block_size;
  const int32_t* heads; int64_t n_heads;
  void* k_coarse; int64_t kc_sb, kc_st, kc_sh;
  void* v_coarse; int64_t vc_sb, vc_st, vc_sh;
  int64_t coarse_cap, c_dst, c_src, c_rows;
} wa_kv_roll_args;
int wa_kv_roll(const wa_kv_roll_args* args, void* stream);

/* Boolean selection mask [rows, ncols] (uint8) -> ascending (index [rows, ncols], num [rows]),
 * index padded with -1. Replaces map_to_index, wan/modules/hsa/block_sparse_triton.py:20-57. */
int wa_map_to_index(const uint8_t* mask, int64_t rows, int64_t ncols, int32_t* index,
                    int32_t* num, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Block-sparse attention                                                                      */
/* ------------------------------------------------------------------------------------------ */

/* Forward of block-sparse flash attention (bf16 q/k/v, fp32 accumulation).
 * Replaces _fwd_kernel/_forward, wan/modules/hsa/block_sparse_triton.py:67-139, 303-320, and the
 * torch gather path block_sparse_attention_reference, block_sparse_torch.py:16-64.
 * Query block i (block_size rows) attends to key blocks index[b,h,i,0:num[b,h,i]] (ids clamped
 * to [0, Nkv-1]); key tokens past min(block_sizes[j], Lkv - j*block_size) are masked; a row with
 * num = 0 yields 0 (and lse = -inf). index == NULL selects every key block (dense attention).
 * heads (optional): device int32[n_heads], the heads to attend (head slots 0 .. n_heads - 1);
 * NULL with n_heads = 0 = all H heads (NULL with n_heads > 0 is an error).
 * lse (optional): [B, H, Lq] natural-log log-sum-exp of the scaled logits.
 * Epilogue (per element, gate g = sigmoid(q . gate_w[d] + gate_b[d]) or sigmoid(q) when gate_w
 * is NULL, optionally rounded to bf16 before/after the sigmoid):
 *   PLAIN: o = attn;  FUSE: o = attn + g * x;  GATED: o = g * attn
 * — the gated fusion of attention.py:246-254 done in registers.
 *
 * Work is split into units of at most split_visits consecutive list entries (0 = the default:
 * WA_BSA_DEFAULT_SPLIT for 128-key blocks, WA_BSA_DEFAULT_SPLIT_64 for 64-key blocks) per
 * (row = b, head, query block). A row with one unit is written by it; the units of a longer row
 * leave normalized partials in `workspace`, and the row's last unit to finish merges them in split
 * order (results do not depend on scheduling). max_visits (0 = index_width) must bound every
 * row's num: visits past max_visits are not computed. units (optional, device int32
 * [n_units][2] = (row, split)) lists the units to launch, in launch order; it must contain every
 * split of every row with num > 0 and split 0 of every row with num = 0, which writes that row
 * (rows are numbered (b * n_heads + head_slot) * Nq + i). Without it every
 * (row, split < max(1, ceil(max_visits / split_visits))) is launched.
 * arrivals (optional): [rows] int32 counters the units use to find each row's last unit; they
 * must be 0 on entry (e.g. cleared by wa_route's `clear`, or left so by the previous launch that
 * used them) and are 0 again when the launch completes. NULL: the launch clears counters in
 * `workspace` with one extra small kernel (none when every row takes a single unit, which counts
 * nothing). Launches that overlap must not share arrivals. */
#define WA_BSA_DEFAULT_SPLIT 16
#define WA_BSA_DEFAULT_SPLIT_64 48
typedef struct wa_bsa_fwd_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  void* o; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  float* lse;
  const int32_t* index; const int32_t* num; int64_t index_width;
  const int32_t* block_sizes;
  const int32_t* heads; int64_t n_heads;
  int64_t B, H, Lq, Lkv, D, block_size;
  float scale;
  int32_t epilogue;
  const void* x; int64_t x_sb, x_st, x_sh; int32_t x_dtype;
  const void* gate_w; const float* gate_b;
  int32_t gate_pre_bf16, gate_out_bf16, attn_round_bf16;
  void* workspace;
  const int32_t* units; int64_t n_units;
  int64_t max_visits; int32_t split_visits;
  int32_t* arrivals;
} wa_bsa_fwd_args;
/* Workspace bytes for rows = B * n_heads * ceil(Lq / block_size) rows. */
int64_t wa_bsa_fwd_workspace_bytes(int64_t rows, int64_t max_visits, int64_t split_visits, int64_t block_size,
                                   int64_t D);
int wa_bsa_fwd(const wa_bsa_fwd_args* args, void* stream);

/* wa_bsa_fwd that allocates nothing and takes no workspace. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The split partials and arrival counters live in a
 * static device array of the library, WA_BSA_FWD_NOALLOC_SCRATCH_BYTES per GPU, held from the
 * library's first use on that GPU until the process ends. args->workspace and args->arrivals must
 * be NULL; a launch whose wa_bsa_fwd_workspace_bytes exceeds the array is rejected (WA_ERR_ARG)
 * before anything runs. The counters are cleared by a fill kernel at the start of every call. All
 * calls on one GPU share its array, so calls that overlap on one GPU (on different streams) race;
 * calls in one stream are ordered and safe. Results equal wa_bsa_fwd's bit for bit. */
#define WA_BSA_FWD_NOALLOC_SCRATCH_BYTES (64ll << 20)
int wa_bsa_fwd_noalloc(const wa_bsa_fwd_args* args, void* stream);

/* The HSA forward of heads that take one branch each, in one call: block pooling of the sparse
 * heads' queries and keys (wa_block_mean_pool_n), their top-k routing (wa_route, TOPK; index / num
 * written for the caller), the block-sparse attention of those heads rounded to bf16 (wa_bsa_fwd,
 * PLAIN), the elu(x)+1 state of the linear heads (wa_elu1_state) and their gated readout
 * (wa_elu1_readout, GATED), from one workspace of wa_hsa_fwd_workspace_bytes.
 * It replaces the orchestration of hsa_attention, wan/modules/hsa/attention.py:153-259, for the
 * north-star head modes (sparse / linear heads, no head in both branches) with bf16 q / k / v;
 * the result equals those calls made one by one.
 * head_k: [H] top-k budget per global head. units / n_units / max_visits: the unit table of the
 * sparse launch (see wa_bsa_fwd).
 * side_stream / fork_event / join_event (hipStream_t / hipEvent_t, owned by the caller): with a
 * side stream and both kinds of head, the two elu1 calls run on it, concurrently with the sparse
 * heads on `stream`: the call records fork_event on `stream` and makes the side stream wait for
 * it, and at its end records join_event on the side stream and makes `stream` wait for it (so a
 * graph captured from `stream` holds both branches). NULL side_stream: everything runs on
 * `stream`. The call keeps no state and takes no lock; concurrent calls need their own side
 * stream and events.
 * Training outputs (all optional; NULL for an inference call), what wa_hsa_bwd takes back:
 * lse: [B, H, Lq] fp32 natural-log log-sum-exp of the sparse heads (wa_bsa_fwd's lse);
 * state / zsum: where the elu1 state of the linear heads goes ([B, n_linear, D, D] and
 * [B, n_linear, D] fp32; NULL: the workspace);
 * lin / gate (fp32 BLHD, given together with lin_modes, a device int32[H] of head modes, 2 for a
 * linear head and 0 otherwise): the linear heads' readout is written unfused into lin
 * (wa_elu1_readout, PLAIN) and wa_hsa_fuse_fwd forms their gate (into gate) and output, as the
 * autograd forward does (the output is the same as the GATED readout's). */
typedef struct wa_hsa_fwd_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  void* o; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  int64_t B, H, Lq, Lkv, D, block_size;
  const int32_t* sparse_heads; int64_t n_sparse;
  const int32_t* head_k;
  const int32_t* units; int64_t n_units; int64_t max_visits;
  int32_t* index; int32_t* num;
  const int32_t* linear_heads; int64_t n_linear;
  const void* gate_w; const float* gate_b;
  int32_t gate_pre_bf16, gate_out_bf16, lin_round_bf16;
  void* workspace;
  void* side_stream; void* fork_event; void* join_event;
  float* lse;
  float* state; float* zsum;
  float* lin; int64_t lin_sb, lin_st, lin_sh;
  float* gate; int64_t gate_sb, gate_st, gate_sh;
  const int32_t* lin_modes;
} wa_hsa_fwd_args;
int64_t wa_hsa_fwd_workspace_bytes(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D, int64_t block_size,
                                   int64_t n_sparse, int64_t n_linear, int64_t max_visits);
int wa_hsa_fwd(const wa_hsa_fwd_args* args, void* stream);

/* The HSA backward of heads that take one branch each, in one call: the gradients of wa_hsa_fwd's
 * output (given its training outputs lse, state, zsum, lin and gate, its routing index / num, and
 * the sparse heads' output o, which the forward wrote rounded to bf16 into its output).
 * Sparse heads: wa_bsa_bwd (dq, dk, dv written). Linear heads: wa_hsa_fuse_bwd (dlin = dout * gate
 * into the workspace, the gate path written into dq, dgate_w / dgate_b written when gate_w is
 * given) then wa_elu1_bwd (added into dq; dk, dv written). Every gradient element of a listed
 * head is written (no accumulation, no prior fill needed); unlisted heads are not touched.
 * dq: fp32 or bf16 (dq_dtype; bf16: the sparse heads' dq kernel rounds its fp32 result once, the
 * linear heads' fp32 sum in the workspace is rounded by a final pass). dk / dv: fp32 or bf16
 * (dkv_dtype). side_stream / fork_event / join_event as in wa_hsa_fwd: the linear heads run on
 * the side stream, concurrently with the sparse heads. Results equal those calls made one by one.
 * Replaces the autograd of hsa_attention (wan/modules/hsa/attention.py:153-259) with the Triton
 * backward, wan/modules/hsa/block_sparse_triton.py:353-368, for the north-star head modes. */
typedef struct wa_hsa_bwd_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  const void* o; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  const void* dout; int64_t d_sb, d_st, d_sh; int32_t dout_dtype;
  int64_t B, H, Lq, Lkv, D, block_size;
  const int32_t* sparse_heads; int64_t n_sparse;
  const int32_t* index; const int32_t* num;
  const float* lse;
  const int32_t* linear_heads; int64_t n_linear;
  const int32_t* lin_modes;
  const float* lin; int64_t lin_sb, lin_st, lin_sh;
  const float* gate; int64_t gate_sb, gate_st, gate_sh;
  const float* state; const float* zsum;
  const void* gate_w; const float* gate_b;
  int32_t gate_pre_bf16, gate_out_bf16, lin_round_bf16;
  void* dq; int64_t dq_sb, dq_st, dq_sh; int32_t dq_dtype;
  void* dk; int64_t dk_sb, dk_st, dk_sh;
  void* dv; int64_t dv_sb, dv_st, dv_sh; int32_t dkv_dtype;
  float* dgate_w; float* dgate_b;
  void* workspace;
  void* side_stream; void* fork_event; void* join_event;
  /* dq_stream / dq_fork_event / dq_join_event (optional, caller-owned, another stream than the two
   * above): the sparse heads' dQ pass runs there, forked after their preprocess, concurrently with
   * their dK/dV pass (and the linear heads), and joined back before the call returns. */
  void* dq_stream; void* dq_fork_event; void* dq_join_event;
} wa_hsa_bwd_args;
int64_t wa_hsa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Lq, int64_t Lkv, int64_t D, int64_t block_size,
                                   int64_t n_sparse, int64_t n_linear);
int wa_hsa_bwd(const wa_hsa_bwd_args* args, void* stream);

/* Backward of wa_bsa_fwd: dQ, dK, dV (fp32, BLHD) of the block-sparse attention output o.
 * Replaces _bwd_preprocess/_bwd_kernel/_backward, wan/modules/hsa/block_sparse_triton.py:142-368
 * (which requires Lq == Lkv), and the autograd of block_sparse_torch.py:16-64: any Lq / Lkv, a
 * key block listed twice contributes twice, masked keys and empty rows contribute nothing.
 * o: the forward's attention output (fp32 preferred; its row dot product with dout is delta),
 * dout: gradient of o, lse: the forward's natural-log log-sum-exp [B, H, Lq]. index / num /
 * block_sizes / heads as in wa_bsa_fwd. dq (optional), dk + dv (optional pair): with
 * *_accumulate set the gradient is added to the existing contents. dk / dv are fp32, or bf16
 * (rounded to nearest even) when dkv_dtype = WA_BF16, which requires both accumulate flags off
 * (a bf16 gradient is written once, in its final type). Routing is not
 * differentiated. Work: a preprocess pass, the transposed (key block -> query blocks) lists,
 * a dQ pass over each query block's list and a dK/dV pass over each key block's list; sums run
 * in a fixed order (reproducible). */
typedef struct wa_bsa_bwd_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  const void* o; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  const void* dout; int64_t d_sb, d_st, d_sh; int32_t dout_dtype;
  const float* lse;
  const int32_t* index; const int32_t* num; int64_t index_width;
  const int32_t* block_sizes;
  const int32_t* heads; int64_t n_heads;
  int64_t B, H, Lq, Lkv, D, block_size;
  float scale;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int32_t dq_accumulate;
  void* dk; int64_t dk_sb, dk_st, dk_sh; int32_t dk_accumulate;
  void* dv; int64_t dv_sb, dv_st, dv_sh; int32_t dv_accumulate;
  void* workspace;
  int32_t dkv_dtype;  /* WA_F32 or WA_BF16 */
  int32_t dq_dtype;   /* WA_F32, or WA_BF16 (rounded to nearest even once; requires dq_accumulate off) */
} wa_bsa_bwd_args;
int64_t wa_bsa_bwd_workspace_bytes(int64_t B, int64_t n_heads, int64_t Lq, int64_t Lkv, int64_t D,
                                   int64_t block_size);
int wa_bsa_bwd(const wa_bsa_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Linear branch                                                                               */
/* ------------------------------------------------------------------------------------------ */

/* Low-rank sequence projection per segment: for each segment of at most segment_len tokens,
 * out[seg rows] = proj[0:r, 0:seg_len] @ x[seg], r = min(proj_rank, ceil(seg_len/block_size)),
 * fp32 accumulation, output rows concatenated along the token axis (out is BLHD, Lc rows).
 * Replaces compress_kv, wan/modules/hsa/attention.py:64-110. */
typedef struct wa_compress_args {
  const void* x; int64_t x_sb, x_st, x_sh; int32_t x_dtype;
  const void* proj; int32_t proj_dtype; int64_t proj_rank, proj_len;
  int64_t B, L, H, D, segment_len, block_size;
  void* out; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
} wa_compress_args;
int wa_compress_kv(const wa_compress_args* args, void* stream);

/* Backward of wa_compress_kv. dout: gradient of the compressed rows (fp32, BLHD strides, the Lc
 * rows wa_compress_kv wrote); x, proj and the sizes as in the forward, with E = proj's stored
 * values (fp32, or bf16 widened). Per segment (rows row0 .. row0 + r of dout, tokens start ..):
 *   dx[b, start + t, h, :] = sum_j E[j, t] dout[b, row0 + j, h, :]      (fp32; optional)
 *   dproj[j, t] = sum over segments, batches, heads and channels of dout[row0 + j] x[start + t]
 * dproj (optional) is [proj_rank, proj_len] fp32 row-major; entries no segment covers get zero.
 * With *_accumulate set the gradient is added to the existing contents. fp32 arithmetic; the
 * dproj sum runs in a fixed order (per-segment partials in `workspace`, of
 * wa_compress_kv_bwd_workspace_bytes, added in segment order), so results repeat bit for bit.
 * dout and dx are read / written by float4 and x by 16 bytes: each must be 16-byte aligned with
 * strides that keep every row so.
 * Replaces the autograd of compress_kv's per-segment matmul, wan/modules/hsa/attention.py:64-110. */
typedef struct wa_compress_bwd_args {
  const float* dout; int64_t d_sb, d_st, d_sh;
  const void* x; int64_t x_sb, x_st, x_sh; int32_t x_dtype;
  const void* proj; int32_t proj_dtype; int64_t proj_rank, proj_len;
  int64_t B, L, H, D, segment_len, block_size;
  float* dx; int64_t dx_sb, dx_st, dx_sh; int32_t dx_accumulate;
  float* dproj; int32_t dproj_accumulate;
  void* workspace;
} wa_compress_bwd_args;
int64_t wa_compress_kv_bwd_workspace_bytes(int64_t L, int64_t proj_rank, int64_t segment_len, int64_t block_size);
int wa_compress_kv_bwd(const wa_compress_bwd_args* args, void* stream);

/* Kernelized linear attention state (north star, no reference counterpart):
 * state[b,s,d,e] = sum_t v[t,d] * phi(k[t,e]) and zsum[b,s,e] = sum_t phi(k[t,e]) with
 * phi(x) = elu(x) + 1, for each listed head heads[s] (fp32 outputs, [B, n_heads, D, D] / [B, n_heads, D]);
 * D in {64, 128}, k/v bf16 or fp32. Chunk partials are summed in a fixed order (reproducible). */
typedef struct wa_elu1_state_args {
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh;
  int32_t dtype;
  int64_t B, H, L, D;
  const int32_t* heads; int64_t n_heads;
  float* state; float* zsum;
  void* workspace;
} wa_elu1_state_args;
int64_t wa_elu1_state_workspace_bytes(int64_t B, int64_t n_heads, int64_t L, int64_t D);
int wa_elu1_state(const wa_elu1_state_args* args, void* stream);

/* Kernelized linear attention readout: o[t] = phi(q[t]) S / (phi(q[t]) . z) per listed head,
 * with the same epilogue options as wa_bsa_fwd (GATED: o = g * o_lin). */
typedef struct wa_elu1_readout_args {
  const void* q; int64_t q_sb, q_st, q_sh; int32_t q_dtype;
  const float* state; const float* zsum;
  void* o; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  int64_t B, H, L, D;
  const int32_t* heads; int64_t n_heads;
  int32_t epilogue;
  const void* gate_w; const float* gate_b;
  int32_t gate_pre_bf16, gate_out_bf16, lin_round_bf16;
} wa_elu1_readout_args;
int wa_elu1_readout(const wa_elu1_readout_args* args, void* stream);

/* Backward of the elu(x)+1 linear branch (wa_elu1_state + PLAIN wa_elu1_readout): given the
 * forward's state / zsum and dout = dL/d(readout output), writes fp32 dq and fp32 or bf16
 * (dkv_dtype) dk, dv (BLHD; with *_accumulate set, added to the contents; bf16 only without) for
 * the listed heads. No reference counterpart (the
 * north-star linear heads); the query-tile partial sums of dS and dz are reduced in a fixed order. */
typedef struct wa_elu1_bwd_args {
  const void* q; int64_t q_sb, q_st, q_sh; int32_t q_dtype;
  const void* k; int64_t k_sb, k_st, k_sh;
  const void* v; int64_t v_sb, v_st, v_sh; int32_t kv_dtype;
  const void* dout; int64_t d_sb, d_st, d_sh; int32_t dout_dtype;
  const float* state; const float* zsum;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int32_t dq_accumulate;
  void* dk; int64_t dk_sb, dk_st, dk_sh; int32_t dk_accumulate;
  void* dv; int64_t dv_sb, dv_st, dv_sh; int32_t dv_accumulate;
  const int32_t* heads; int64_t n_heads;
  int64_t B, H, Lq, Lkv, D;
  void* workspace;
  int32_t dkv_dtype;  /* WA_F32 or WA_BF16 (then both kv accumulate flags must be off) */
} wa_elu1_bwd_args;
int64_t wa_elu1_bwd_workspace_bytes(int64_t B, int64_t n_heads, int64_t Lq, int64_t D);
int wa_elu1_bwd(const wa_elu1_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Gated fusion as separate kernels (training path)                                            */
/* ------------------------------------------------------------------------------------------ */

/* Branch fusion of attention.py:246-254 with per-head modes (head_modes[h]: bit 0 = the head runs
 * the sparse branch, bit 1 = the linear branch, 0 = not written):
 *   gate = sigmoid(q . gate_w[d] + gate_b[d])  (sigmoid(q) when gate_w is NULL; bf16 rounding of
 *          the pre-activation / gate per the flags, as the reference's dtype casts do),
 *   out  = [sparse] + [gate * linear]   (sparse / linear fp32 BLHD, optionally rounded to bf16).
 * wa_hsa_fuse_fwd writes out and, when `gate` is given, the gate values of linear heads.
 * wa_hsa_fuse_bwd takes dout, lin and the saved gate and writes dlin = dout * gate, adds
 * dgpre * gate_w (or dgpre) into dq, and with gate_w writes dgate_w [D][D] and dgate_b [D]
 * (sums of per-tile partials, fixed order; workspace from wa_hsa_fuse_bwd_workspace_bytes). The
 * sparse branch's gradient is dout itself. q is bf16 BLHD. */
typedef struct wa_hsa_fuse_args {
  const void* q; int64_t q_sb, q_st, q_sh;
  const float* sparse; int64_t s_sb, s_st, s_sh;
  const float* lin; int64_t l_sb, l_st, l_sh;
  const int32_t* head_modes;
  void* out; int64_t o_sb, o_st, o_sh; int32_t o_dtype;
  float* gate; int64_t g_sb, g_st, g_sh;
  const void* gate_w; const float* gate_b;
  int32_t gate_pre_bf16, gate_out_bf16, attn_round_bf16, lin_round_bf16;
  const void* dout; int64_t d_sb, d_st, d_sh; int32_t dout_dtype;
  float* dlin; int64_t dl_sb, dl_st, dl_sh;
  float* dq; int64_t dq_sb, dq_st, dq_sh; int32_t dq_accumulate;
  float* dgate_w; float* dgate_b;
  void* workspace;
  int64_t B, H, L, D;
} wa_hsa_fuse_args;
int wa_hsa_fuse_fwd(const wa_hsa_fuse_args* args, void* stream);
int64_t wa_hsa_fuse_bwd_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t D);
int wa_hsa_fuse_bwd(const wa_hsa_fuse_args* args, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* HKV tier: page summaries, page selection, temporal re-rotation, host-tier copies             */
/* ------------------------------------------------------------------------------------------ */

/* Segment means of a [B, T, C] tensor (C = H*D; element (b, t, c) at x + b*x_sb + t*x_st + c) into
 * fp32 out[n_seg][C]:  out[s][c] = mean_b ( mean_{t in segment s} y[b][t][c] ).
 * Segment s is [s*seg_tokens, min((s+1)*seg_tokens, T)), or [spans[2s], spans[2s+1]) when `spans`
 * (device int32 [n_seg][2]) is given; max_seg_tokens bounds every segment's length.
 * With `factors` (device complex64 as float pairs, [n_rows][n_temporal]), y is x with complex pair
 * p < n_temporal of every head multiplied by factors[min(t / row_tokens, n_rows - 1)][p] in fp32
 * and rounded to x's dtype (the reference de-ropes into the cache dtype, then pools in fp32);
 * without `factors`, y = x. With `normalize`, each out row becomes row / max(|row|_2, 1e-12).
 * Replaces page_key_index + derope_temporal (pipeline/hkv/retrieval.py:50-72, rope.py:70-82),
 * query_index (retrieval.py:41-47) and prompt_index (retrieval.py:32-38, normalize = 1).
 * Workspace: wa_hkv_summary_workspace_bytes(B, n_seg, C, max_seg_tokens). */
typedef struct wa_hkv_summary_args {
  const void* x; int64_t x_sb, x_st; int32_t x_dtype;
  int64_t B, T, H, D;
  int64_t seg_tokens; const int32_t* spans; int64_t n_seg; int64_t max_seg_tokens;
  const float* factors; int64_t n_temporal, row_tokens, n_rows;
  int32_t normalize;
  float* out;
  void* workspace;
} wa_hkv_summary_args;
int64_t wa_hkv_summary_workspace_bytes(int64_t B, int64_t n_seg, int64_t C, int64_t max_seg_tokens);
int wa_hkv_page_summary(const wa_hkv_summary_args* args, void* stream);

/* Page scoring and selection in one workgroup:
 *   scores[p] = (index[p] . query) / scale   (no division when scale <= 0), p < n_pages <= 4096,
 * then the k highest in descending order, the lower page index first among equal scores (NaN
 * ranks highest), into sel (int32) and sel_scores. Pages with mask[p] != 0 (device uint8,
 * optional) are never selected; slots beyond the unmasked count get sel = -1, score = -inf.
 * Replaces score_pages + select_topk_pages (pipeline/hkv/retrieval.py:75-89, 105-126) and the
 * stage-1 cosine ranking select_top_chunks (retrieval.py:92-102, scale = 0). */
#define WA_HKV_MAX_PAGES 4096
typedef struct wa_hkv_topk_args {
  const float* index; int64_t index_stride;   /* [n_pages][dim] fp32 */
  const float* query;                          /* [dim] fp32 */
  int64_t n_pages, dim;
  float scale;
  const uint8_t* mask;
  int64_t k;
  float* scores;                               /* optional [n_pages] */
  int32_t* sel; float* sel_scores;             /* [k] each */
} wa_hkv_topk_args;
int wa_hkv_score_topk(const wa_hkv_topk_args* args, void* stream);

/* Temporal re-rotation of tokens [t0, t1) of a BLHD tensor: complex pair p < n_temporal of every
 * head is multiplied by factors[row][p] (complex64 as float pairs, fp32 math) and rounded to the
 * tensor's dtype, row = rows[t - t0] (device int32) when `rows` is given, else
 * min((t - t0) / row_tokens, n_rows - 1). src == dst rotates in place (only the temporal band is
 * read and written); otherwise every channel is copied to dst (same dtype). Replaces
 * shift_temporal_rope (pipeline/hkv/rope.py:50-67, one factor per installed page at
 * cache.py:229-238 with the moves of cache.py:273-286) and derope_temporal (rope.py:70-82). */
typedef struct wa_rerope_args {
  const void* src; int64_t s_sb, s_st, s_sh;
  void* dst; int64_t d_sb, d_st, d_sh;
  int32_t dtype;
  int64_t B, t0, t1, H, D;
  const float* factors; int64_t n_temporal, n_rows;
  const int32_t* rows; int64_t row_tokens;
} wa_rerope_args;
int wa_rerope(const wa_rerope_args* args, void* stream);

/* Host-tier copies: each is `rows` rows of `width` bytes at the given pitches, enqueued in order
 * on `stream` (hipMemcpy2DAsync); `done` (hipEvent_t, optional) is recorded after the last one.
 * The host side must be pinned (hipHostMalloc / torch pin_memory) and is checked.
 * wa_hkv_gather_async: pinned host -> device, the page install of HKVCache.apply
 *   (pipeline/hkv/cache.py:229-246, which copies page by page with synchronous .to(device));
 * wa_hkv_store_async: device -> pinned host, the chunk store of HKVCache.store (cache.py:104-107,
 *   pageable .to("cpu")). */
typedef struct wa_hkv_copy {
  const void* src; int64_t src_pitch;
  void* dst; int64_t dst_pitch;
  int64_t width, rows;
} wa_hkv_copy;
int wa_hkv_gather_async(const wa_hkv_copy* copies, int64_t n, void* stream, void* done);
int wa_hkv_store_async(const wa_hkv_copy* copies, int64_t n, void* stream, void* done);

/* Asynchronous file I/O of the HKV NVMe tier: replaces the synchronous torch.save / torch.load of a
 * spilled chunk (pipeline/hkv/tiering.py:89-105). wa_io_write_async / wa_io_read_async move the n
 * host buffers (bufs[i], sizes[i] bytes) to / from the file at `path`, buffer i at the 4 KiB-aligned
 * offset sum(round_up(sizes[j], 4096), j < i), on a worker thread, with O_DIRECT when `direct` is
 * set and the file system takes it (buffered I/O otherwise; page-aligned buffers go to the device
 * directly, the rest through an aligned bounce buffer). The file is opened (created, for a write)
 * before the call returns; the buffers must stay valid until wa_io_wait. Returns a handle > 0, or
 * a negative status. wa_io_done: 1 when the transfer has finished, 0 while it runs;
 * wa_io_direct: 1 if O_DIRECT is in use; wa_io_wait: joins the transfer and releases the handle
 * (WA_OK, or WA_ERR_IO with the reason in wa_last_error). No reference counterpart beyond the
 * tier's spill / reload. */
int64_t wa_io_write_async(const char* path, const void* const* bufs, const int64_t* sizes, int64_t n, int32_t direct);
int64_t wa_io_read_async(const char* path, void* const* bufs, const int64_t* sizes, int64_t n, int32_t direct);
int wa_io_done(int64_t handle);
int wa_io_direct(int64_t handle);
int wa_io_wait(int64_t handle);

/* Page install with the re-rope fused in: replaces the page-by-page install + rotation of
 * HKVCache.apply (pipeline/hkv/cache.py:229-246, shift_temporal_rope per page at :233-238). Each
 * page (a pinned host [B, tokens, H, D] view, element strides) is read by a kernel through its
 * device mapping and written to cache tokens [dst_token, dst_token + tokens) of `dst`
 * ([B, cap, H, D] on the device), its temporal band (complex pairs < n_temporal) multiplied by
 * factor row i of `factors` ([n_pages, n_temporal] complex fp32 as (re, im) pairs, device; NULL:
 * plain copy) as wa_rerope does, so the installed keys need no second pass over HBM. Pages must
 * stay alive until the stream passes the launch. */
typedef struct wa_hkv_page {
  const void* src; int64_t s_sb, s_st, s_sh;
  int64_t tokens, dst_token;
} wa_hkv_page;
typedef struct wa_hkv_gather_rotate_args {
  const wa_hkv_page* pages; int64_t n_pages;
  void* dst; int64_t d_sb, d_st, d_sh;
  int32_t dtype;
  int64_t B, cap, H, D;
  const float* factors; int64_t n_temporal;
} wa_hkv_gather_rotate_args;
int wa_hkv_gather_rotate(const wa_hkv_gather_rotate_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WORLDATTENTION_AMD_H */
