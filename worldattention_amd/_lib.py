"""ctypes binding of ``libworldattention_amd.so`` (declared in ``include/worldattention_amd.h``).

The library is the only compute path: if it is missing, or a tensor is not on a ROCm GPU, the
calls raise — there is no CPU fallback. Argument structs mirror the C header field for field.
"""
from __future__ import annotations

import ctypes
import functools
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p

import torch

# WORLDATTENTION_AMD_LIB selects another build of the library (e.g. to compare two builds); the
# default is the in-tree build next to this file
LIB_PATH = os.environ.get("WORLDATTENTION_AMD_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                   "libworldattention_amd.so")

WA_OK, WA_ERR_ARG, WA_ERR_UNSUPPORTED, WA_ERR_IO = 0, -1, -2, -3
WA_F32, WA_BF16 = 0, 1
WA_ROUTE_GINI, WA_ROUTE_TOPK = 0, 1
WA_EPI_PLAIN, WA_EPI_FUSE, WA_EPI_GATED = 0, 1, 2


def _struct(name, fields):
    return type(name, (ctypes.Structure,), {"_fields_": fields})


PoolArgs = _struct("wa_pool_args", [
    ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_sh", c_int64), ("x_dtype", c_int32),
    ("B", c_int64), ("L", c_int64), ("H", c_int64), ("D", c_int64), ("block_size", c_int64),
    ("num_blocks", c_int64), ("heads", c_void_p), ("n_heads", c_int64), ("out", c_void_p),
    ("emulate_rounding", c_int32),
    ("first_block", c_int64), ("out_blocks", c_int64), ("store_sums", c_int32),
])

RouteArgs = _struct("wa_route_args", [
    ("probs", c_void_p), ("q_pooled", c_void_p), ("k_pooled", c_void_p),
    ("B", c_int64), ("H", c_int64), ("Nq", c_int64), ("Nkv", c_int64), ("D", c_int64),
    ("mode", c_int32), ("tau_min", c_float), ("tau_span", c_float),
    ("head_k", c_void_p), ("heads", c_void_p), ("n_heads", c_int64),
    ("index", c_void_p), ("num", c_void_p), ("thresholds", c_void_p), ("mask", c_void_p),
    ("probs_out", c_void_p), ("workspace", c_void_p), ("clear", c_void_p), ("n_clear", c_int64),
    ("k_sum_len", c_int64), ("block_size", c_int64), ("k_sum_bf16", c_int32),
    ("k_pooled_blocks", c_int64), ("scale", c_float),
])

KvAppendArgs = _struct("wa_kv_append_args", [
    ("cache_k", c_void_p), ("ck_sb", c_int64), ("ck_st", c_int64), ("ck_sh", c_int64),
    ("cache_v", c_void_p), ("cv_sb", c_int64), ("cv_st", c_int64), ("cv_sh", c_int64),
    ("new_k", c_void_p), ("nk_sb", c_int64), ("nk_st", c_int64), ("nk_sh", c_int64),
    ("new_v", c_void_p), ("nv_sb", c_int64), ("nv_st", c_int64), ("nv_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("cap", c_int64), ("H", c_int64), ("D", c_int64), ("start", c_int64), ("n", c_int64),
    ("k_sums", c_void_p), ("block_size", c_int64),
    ("heads", c_void_p), ("n_heads", c_int64),
])

QkvEpilogueArgs = _struct("wa_qkv_epilogue_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("n", c_int64), ("H", c_int64), ("D", c_int64),
    ("q_out", c_void_p), ("qo_sb", c_int64), ("qo_st", c_int64), ("qo_sh", c_int64),
    ("cache_k", c_void_p), ("ck_sb", c_int64), ("ck_st", c_int64), ("ck_sh", c_int64),
    ("cache_v", c_void_p), ("cv_sb", c_int64), ("cv_st", c_int64), ("cv_sh", c_int64),
    ("cap", c_int64), ("write_start", c_int64), ("src_offset", c_int64), ("write_len", c_int64),
    ("freqs", c_void_p), ("f_rows", c_int64),
    ("grid_f", c_int64), ("grid_h", c_int64), ("grid_w", c_int64), ("start_frame", c_int64),
    ("q_norm_w", c_void_p), ("k_norm_w", c_void_p), ("w_dtype", c_int32), ("eps", c_float),
    ("k_sums", c_void_p), ("block_size", c_int64),
    ("sample_grids", POINTER(c_int64)),
])

KvRollArgs = _struct("wa_kv_roll_args", [
    ("cache_k", c_void_p), ("ck_sb", c_int64), ("ck_st", c_int64), ("ck_sh", c_int64),
    ("cache_v", c_void_p), ("cv_sb", c_int64), ("cv_st", c_int64), ("cv_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("cap", c_int64), ("H", c_int64), ("D", c_int64),
    ("sink", c_int64), ("evicted", c_int64), ("rolled", c_int64),
    ("k_sums", c_void_p), ("block_size", c_int64),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("k_coarse", c_void_p), ("kc_sb", c_int64), ("kc_st", c_int64), ("kc_sh", c_int64),
    ("v_coarse", c_void_p), ("vc_sb", c_int64), ("vc_st", c_int64), ("vc_sh", c_int64),
    ("coarse_cap", c_int64), ("c_dst", c_int64), ("c_src", c_int64), ("c_rows", c_int64),
])

HkvPage = _struct("wa_hkv_page", [
    ("src", c_void_p), ("s_sb", c_int64), ("s_st", c_int64), ("s_sh", c_int64),
    ("tokens", c_int64), ("dst_token", c_int64),
])

HkvGatherRotateArgs = _struct("wa_hkv_gather_rotate_args", [
    ("pages", c_void_p), ("n_pages", c_int64),
    ("dst", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("cap", c_int64), ("H", c_int64), ("D", c_int64),
    ("factors", c_void_p), ("n_temporal", c_int64),
])

BsaFwdArgs = _struct("wa_bsa_fwd_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("o", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("lse", c_void_p),
    ("index", c_void_p), ("num", c_void_p), ("index_width", c_int64),
    ("block_sizes", c_void_p),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("B", c_int64), ("H", c_int64), ("Lq", c_int64), ("Lkv", c_int64), ("D", c_int64), ("block_size", c_int64),
    ("scale", c_float),
    ("epilogue", c_int32),
    ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_sh", c_int64), ("x_dtype", c_int32),
    ("gate_w", c_void_p), ("gate_b", c_void_p),
    ("gate_pre_bf16", c_int32), ("gate_out_bf16", c_int32), ("attn_round_bf16", c_int32),
    ("workspace", c_void_p), ("units", c_void_p), ("n_units", c_int64),
    ("max_visits", c_int64), ("split_visits", c_int32), ("arrivals", c_void_p),
])

BSA_DEFAULT_SPLIT = 16      # WA_BSA_DEFAULT_SPLIT (128-key blocks)
BSA_DEFAULT_SPLIT_64 = 48   # WA_BSA_DEFAULT_SPLIT_64 (64-key blocks)


def bsa_default_split(block_size: int) -> int:
    """wa_bsa_fwd's default visits per unit for this block size."""
    return BSA_DEFAULT_SPLIT_64 if block_size == 64 else BSA_DEFAULT_SPLIT
BSA_FWD_NOALLOC_SCRATCH_BYTES = 64 << 20   # WA_BSA_FWD_NOALLOC_SCRATCH_BYTES

CompressArgs = _struct("wa_compress_args", [
    ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_sh", c_int64), ("x_dtype", c_int32),
    ("proj", c_void_p), ("proj_dtype", c_int32), ("proj_rank", c_int64), ("proj_len", c_int64),
    ("B", c_int64), ("L", c_int64), ("H", c_int64), ("D", c_int64), ("segment_len", c_int64),
    ("block_size", c_int64),
    ("out", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
])

CompressBwdArgs = _struct("wa_compress_bwd_args", [
    ("dout", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64),
    ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_sh", c_int64), ("x_dtype", c_int32),
    ("proj", c_void_p), ("proj_dtype", c_int32), ("proj_rank", c_int64), ("proj_len", c_int64),
    ("B", c_int64), ("L", c_int64), ("H", c_int64), ("D", c_int64), ("segment_len", c_int64),
    ("block_size", c_int64),
    ("dx", c_void_p), ("dx_sb", c_int64), ("dx_st", c_int64), ("dx_sh", c_int64), ("dx_accumulate", c_int32),
    ("dproj", c_void_p), ("dproj_accumulate", c_int32),
    ("workspace", c_void_p),
])

Elu1StateArgs = _struct("wa_elu1_state_args", [
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("H", c_int64), ("L", c_int64), ("D", c_int64),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("state", c_void_p), ("zsum", c_void_p), ("workspace", c_void_p),
])

Elu1ReadoutArgs = _struct("wa_elu1_readout_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64), ("q_dtype", c_int32),
    ("state", c_void_p), ("zsum", c_void_p),
    ("o", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("B", c_int64), ("H", c_int64), ("L", c_int64), ("D", c_int64),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("epilogue", c_int32),
    ("gate_w", c_void_p), ("gate_b", c_void_p),
    ("gate_pre_bf16", c_int32), ("gate_out_bf16", c_int32), ("lin_round_bf16", c_int32),
])

HsaFwdArgs = _struct("wa_hsa_fwd_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("o", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("B", c_int64), ("H", c_int64), ("Lq", c_int64), ("Lkv", c_int64), ("D", c_int64), ("block_size", c_int64),
    ("sparse_heads", c_void_p), ("n_sparse", c_int64),
    ("head_k", c_void_p),
    ("units", c_void_p), ("n_units", c_int64), ("max_visits", c_int64),
    ("index", c_void_p), ("num", c_void_p),
    ("linear_heads", c_void_p), ("n_linear", c_int64),
    ("gate_w", c_void_p), ("gate_b", c_void_p),
    ("gate_pre_bf16", c_int32), ("gate_out_bf16", c_int32), ("lin_round_bf16", c_int32),
    ("workspace", c_void_p),
    ("side_stream", c_void_p), ("fork_event", c_void_p), ("join_event", c_void_p),
    ("lse", c_void_p), ("state", c_void_p), ("zsum", c_void_p),
    ("lin", c_void_p), ("lin_sb", c_int64), ("lin_st", c_int64), ("lin_sh", c_int64),
    ("gate", c_void_p), ("gate_sb", c_int64), ("gate_st", c_int64), ("gate_sh", c_int64),
    ("lin_modes", c_void_p),
])

HsaBwdArgs = _struct("wa_hsa_bwd_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("o", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("dout", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64), ("dout_dtype", c_int32),
    ("B", c_int64), ("H", c_int64), ("Lq", c_int64), ("Lkv", c_int64), ("D", c_int64), ("block_size", c_int64),
    ("sparse_heads", c_void_p), ("n_sparse", c_int64),
    ("index", c_void_p), ("num", c_void_p),
    ("lse", c_void_p),
    ("linear_heads", c_void_p), ("n_linear", c_int64),
    ("lin_modes", c_void_p),
    ("lin", c_void_p), ("lin_sb", c_int64), ("lin_st", c_int64), ("lin_sh", c_int64),
    ("gate", c_void_p), ("gate_sb", c_int64), ("gate_st", c_int64), ("gate_sh", c_int64),
    ("state", c_void_p), ("zsum", c_void_p),
    ("gate_w", c_void_p), ("gate_b", c_void_p),
    ("gate_pre_bf16", c_int32), ("gate_out_bf16", c_int32), ("lin_round_bf16", c_int32),
    ("dq", c_void_p), ("dq_sb", c_int64), ("dq_st", c_int64), ("dq_sh", c_int64), ("dq_dtype", c_int32),
    ("dk", c_void_p), ("dk_sb", c_int64), ("dk_st", c_int64), ("dk_sh", c_int64),
    ("dv", c_void_p), ("dv_sb", c_int64), ("dv_st", c_int64), ("dv_sh", c_int64), ("dkv_dtype", c_int32),
    ("dgate_w", c_void_p), ("dgate_b", c_void_p),
    ("workspace", c_void_p),
    ("side_stream", c_void_p), ("fork_event", c_void_p), ("join_event", c_void_p),
    ("dq_stream", c_void_p), ("dq_fork_event", c_void_p), ("dq_join_event", c_void_p),
])

BsaBwdArgs = _struct("wa_bsa_bwd_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
    ("o", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("dout", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64), ("dout_dtype", c_int32),
    ("lse", c_void_p),
    ("index", c_void_p), ("num", c_void_p), ("index_width", c_int64),
    ("block_sizes", c_void_p),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("B", c_int64), ("H", c_int64), ("Lq", c_int64), ("Lkv", c_int64), ("D", c_int64), ("block_size", c_int64),
    ("scale", c_float),
    ("dq", c_void_p), ("dq_sb", c_int64), ("dq_st", c_int64), ("dq_sh", c_int64), ("dq_accumulate", c_int32),
    ("dk", c_void_p), ("dk_sb", c_int64), ("dk_st", c_int64), ("dk_sh", c_int64), ("dk_accumulate", c_int32),
    ("dv", c_void_p), ("dv_sb", c_int64), ("dv_st", c_int64), ("dv_sh", c_int64), ("dv_accumulate", c_int32),
    ("workspace", c_void_p),
    ("dkv_dtype", c_int32), ("dq_dtype", c_int32),
])

Elu1BwdArgs = _struct("wa_elu1_bwd_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64), ("q_dtype", c_int32),
    ("k", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
    ("v", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64), ("kv_dtype", c_int32),
    ("dout", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64), ("dout_dtype", c_int32),
    ("state", c_void_p), ("zsum", c_void_p),
    ("dq", c_void_p), ("dq_sb", c_int64), ("dq_st", c_int64), ("dq_sh", c_int64), ("dq_accumulate", c_int32),
    ("dk", c_void_p), ("dk_sb", c_int64), ("dk_st", c_int64), ("dk_sh", c_int64), ("dk_accumulate", c_int32),
    ("dv", c_void_p), ("dv_sb", c_int64), ("dv_st", c_int64), ("dv_sh", c_int64), ("dv_accumulate", c_int32),
    ("heads", c_void_p), ("n_heads", c_int64),
    ("B", c_int64), ("H", c_int64), ("Lq", c_int64), ("Lkv", c_int64), ("D", c_int64),
    ("workspace", c_void_p),
    ("dkv_dtype", c_int32),
])

HsaFuseArgs = _struct("wa_hsa_fuse_args", [
    ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
    ("sparse", c_void_p), ("s_sb", c_int64), ("s_st", c_int64), ("s_sh", c_int64),
    ("lin", c_void_p), ("l_sb", c_int64), ("l_st", c_int64), ("l_sh", c_int64),
    ("head_modes", c_void_p),
    ("out", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64), ("o_dtype", c_int32),
    ("gate", c_void_p), ("g_sb", c_int64), ("g_st", c_int64), ("g_sh", c_int64),
    ("gate_w", c_void_p), ("gate_b", c_void_p),
    ("gate_pre_bf16", c_int32), ("gate_out_bf16", c_int32), ("attn_round_bf16", c_int32), ("lin_round_bf16", c_int32),
    ("dout", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64), ("dout_dtype", c_int32),
    ("dlin", c_void_p), ("dl_sb", c_int64), ("dl_st", c_int64), ("dl_sh", c_int64),
    ("dq", c_void_p), ("dq_sb", c_int64), ("dq_st", c_int64), ("dq_sh", c_int64), ("dq_accumulate", c_int32),
    ("dgate_w", c_void_p), ("dgate_b", c_void_p),
    ("workspace", c_void_p),
    ("B", c_int64), ("H", c_int64), ("L", c_int64), ("D", c_int64),
])

HkvSummaryArgs = _struct("wa_hkv_summary_args", [
    ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_dtype", c_int32),
    ("B", c_int64), ("T", c_int64), ("H", c_int64), ("D", c_int64),
    ("seg_tokens", c_int64), ("spans", c_void_p), ("n_seg", c_int64), ("max_seg_tokens", c_int64),
    ("factors", c_void_p), ("n_temporal", c_int64), ("row_tokens", c_int64), ("n_rows", c_int64),
    ("normalize", c_int32),
    ("out", c_void_p),
    ("workspace", c_void_p),
])

HKV_MAX_PAGES = 4096

HkvTopkArgs = _struct("wa_hkv_topk_args", [
    ("index", c_void_p), ("index_stride", c_int64),
    ("query", c_void_p),
    ("n_pages", c_int64), ("dim", c_int64),
    ("scale", c_float),
    ("mask", c_void_p),
    ("k", c_int64),
    ("scores", c_void_p), ("sel", c_void_p), ("sel_scores", c_void_p),
])

RopeArgs = _struct("wa_rerope_args", [
    ("src", c_void_p), ("s_sb", c_int64), ("s_st", c_int64), ("s_sh", c_int64),
    ("dst", c_void_p), ("d_sb", c_int64), ("d_st", c_int64), ("d_sh", c_int64),
    ("dtype", c_int32),
    ("B", c_int64), ("t0", c_int64), ("t1", c_int64), ("H", c_int64), ("D", c_int64),
    ("factors", c_void_p), ("n_temporal", c_int64), ("n_rows", c_int64),
    ("rows", c_void_p), ("row_tokens", c_int64),
])

HkvCopy = _struct("wa_hkv_copy", [
    ("src", c_void_p), ("src_pitch", c_int64),
    ("dst", c_void_p), ("dst_pitch", c_int64),
    ("width", c_int64), ("rows", c_int64),
])

# name -> (restype, argtypes)
SIGNATURES = {
    "wa_version": (c_int, []),
    "wa_last_error": (c_char_p, []),
    "wa_block_mean_pool": (c_int, [POINTER(PoolArgs), c_void_p]),
    "wa_block_mean_pool_n": (c_int, [POINTER(PoolArgs), c_int32, c_void_p]),
    "wa_route_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "wa_route": (c_int, [POINTER(RouteArgs), c_void_p]),
    "wa_map_to_index": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "wa_kv_append": (c_int, [POINTER(KvAppendArgs), c_void_p]),
    "wa_qkv_epilogue": (c_int, [POINTER(QkvEpilogueArgs), c_void_p]),
    "wa_kv_roll": (c_int, [POINTER(KvRollArgs), c_void_p]),
    "wa_hkv_gather_rotate": (c_int, [POINTER(HkvGatherRotateArgs), c_void_p]),
    "wa_io_write_async": (c_int64, [c_char_p, POINTER(c_void_p), POINTER(c_int64), c_int64, c_int32]),
    "wa_io_read_async": (c_int64, [c_char_p, POINTER(c_void_p), POINTER(c_int64), c_int64, c_int32]),
    "wa_io_done": (c_int, [c_int64]),
    "wa_io_direct": (c_int, [c_int64]),
    "wa_io_wait": (c_int, [c_int64]),
    "wa_bsa_fwd_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64]),
    "wa_bsa_fwd": (c_int, [POINTER(BsaFwdArgs), c_void_p]),
    "wa_bsa_fwd_noalloc": (c_int, [POINTER(BsaFwdArgs), c_void_p]),
    "wa_compress_kv": (c_int, [POINTER(CompressArgs), c_void_p]),
    "wa_compress_kv_bwd_workspace_bytes": (c_int64, [c_int64] * 4),
    "wa_compress_kv_bwd": (c_int, [POINTER(CompressBwdArgs), c_void_p]),
    "wa_elu1_state_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64]),
    "wa_elu1_state": (c_int, [POINTER(Elu1StateArgs), c_void_p]),
    "wa_elu1_readout": (c_int, [POINTER(Elu1ReadoutArgs), c_void_p]),
    "wa_hsa_fwd_workspace_bytes": (c_int64, [c_int64] * 9),
    "wa_hsa_fwd": (c_int, [POINTER(HsaFwdArgs), c_void_p]),
    "wa_hsa_bwd_workspace_bytes": (c_int64, [c_int64] * 8),
    "wa_hsa_bwd": (c_int, [POINTER(HsaBwdArgs), c_void_p]),
    "wa_bsa_bwd_workspace_bytes": (c_int64, [c_int64] * 6),
    "wa_bsa_bwd": (c_int, [POINTER(BsaBwdArgs), c_void_p]),
    "wa_elu1_bwd_workspace_bytes": (c_int64, [c_int64] * 4),
    "wa_elu1_bwd": (c_int, [POINTER(Elu1BwdArgs), c_void_p]),
    "wa_hsa_fuse_fwd": (c_int, [POINTER(HsaFuseArgs), c_void_p]),
    "wa_hsa_fuse_bwd_workspace_bytes": (c_int64, [c_int64] * 4),
    "wa_hsa_fuse_bwd": (c_int, [POINTER(HsaFuseArgs), c_void_p]),
    "wa_hkv_summary_workspace_bytes": (c_int64, [c_int64] * 4),
    "wa_hkv_page_summary": (c_int, [POINTER(HkvSummaryArgs), c_void_p]),
    "wa_hkv_score_topk": (c_int, [POINTER(HkvTopkArgs), c_void_p]),
    "wa_rerope": (c_int, [POINTER(RopeArgs), c_void_p]),
    "wa_hkv_gather_async": (c_int, [POINTER(HkvCopy), c_int64, c_void_p, c_void_p]),
    "wa_hkv_store_async": (c_int, [POINTER(HkvCopy), c_int64, c_void_p, c_void_p]),
}


@functools.lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise with build instructions when it is absent."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"worldattention_amd: {LIB_PATH} is missing; build it with "
            "`python -m worldattention_amd.csrc.build` (hipcc, gfx950)")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().wa_last_error().decode(errors="replace")
        if rc == WA_ERR_IO:
            raise OSError(f"{name}: {msg}")
        if rc < 0:
            raise ValueError(f"{name}: {msg}")
        raise RuntimeError(f"{name} failed (hip error {rc}): {msg}")


# ----------------------------------------------------------------------------------------------
# tensor helpers
# ----------------------------------------------------------------------------------------------
def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm GPU; there is no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "worldattention_amd runs its HIP kernels on a ROCm GPU only; got a tensor on "
                f"{t.device}. Move inputs to the GPU (there is no CPU fallback).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return WA_BF16
    if t.dtype == torch.float32:
        return WA_F32
    raise TypeError(f"unsupported dtype {t.dtype}; expected bfloat16 or float32")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


def heads_arg(t):
    """``(pointer, count)`` of an optional device head list for the C ABI, where NULL means every
    head. An empty list is refused: its data pointer can be NULL, which the library would read as
    every head while the caller's outputs hold none."""
    if t is None:
        return None, 0
    if t.numel() == 0:
        raise ValueError("empty head list (the library reads a missing list as every head): skip the call")
    return t.data_ptr(), t.numel()


def blhd(t: torch.Tensor):
    """(ptr, sb, st, sh) of a [B, L, H, C] tensor whose channel dim is contiguous."""
    if t.stride(-1) != 1:
        raise ValueError("channel dimension must be contiguous")
    return t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)


def bhld(t: torch.Tensor):
    """(ptr, sb, st, sh) of a [B, H, L, C] tensor (reference sparse-kernel layout)."""
    if t.stride(-1) != 1:
        raise ValueError("channel dimension must be contiguous")
    return t.data_ptr(), t.stride(0), t.stride(2), t.stride(1)


def kernel_ready(t: torch.Tensor, dtype=torch.bfloat16, align_elems: int = 8) -> torch.Tensor:
    """Cast to ``dtype`` and make the channel dim contiguous with 16-byte aligned rows."""
    if t.dtype != dtype:
        t = t.to(dtype)
    if t.stride(-1) != 1 or any(s % align_elems for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
        if t.data_ptr() % 16 or any(s % align_elems for s in t.stride()[:-1]):
            t = t.clone(memory_format=torch.contiguous_format)
    return t


def is_kernel_ready(t: torch.Tensor, dtype=torch.bfloat16, align_elems: int = 8) -> bool:
    """Whether :func:`kernel_ready` would return ``t`` itself (no cast, no copy)."""
    return (t.dtype == dtype and t.stride(-1) == 1 and not any(s % align_elems for s in t.stride()[:-1])
            and t.data_ptr() % 16 == 0)


_HEAD_CACHE: dict = {}


def head_list(heads, device: torch.device) -> torch.Tensor:
    """Device int32 tensor of a small host int list (head ids, per-head budgets), cached per value."""
    key = (str(device), tuple(int(h) for h in heads))
    t = _HEAD_CACHE.get(key)
    if t is None:
        t = torch.tensor(key[1], dtype=torch.int32, device=device)
        _HEAD_CACHE[key] = t
    return t
