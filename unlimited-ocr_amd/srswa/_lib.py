"""ctypes binding of libsrswa.so (C ABI declared in include/srswa.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already holds (one runtime per process; torch's stream handles
are then valid inside the library).  There is no CPU fallback: a missing or
unloadable library raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsrswa.so")

SRSWA_OK = 0
SRSWA_UNSUPPORTED = 1
SRSWA_INVALID = 2
SRSWA_WORKSPACE = 3
SRSWA_LAUNCH = 4

SRSWA_F32 = 0
SRSWA_BF16 = 1
SRSWA_F16 = 2

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p
_szp = ctypes.POINTER(ctypes.c_size_t)


class DecodeArgs(ctypes.Structure):
    """Mirror of ``srswa_decode_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_sq", _i64), ("q_sh", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("v", _vp), ("v_sb", _i64), ("v_st", _i64), ("v_sh", _i64),
        ("idx", _vp), ("idx_sb", _i64), ("idx_sh", _i64), ("idx_sq", _i64), ("idx_ss", _i64),
        ("bias", _vp),
        ("valid", _vp),
        ("q_pos", _vp), ("pos_sb", _i64), ("pos_sq", _i64),
        ("kv_len", _vp),
        ("out", _vp), ("o_sb", _i64), ("o_sq", _i64), ("o_sh", _i64),
        ("lse", _vp), ("lse_sb", _i64), ("lse_sq", _i64), ("lse_sh", _i64),
        ("B", _i32), ("Lq", _i32), ("HQ", _i32), ("HKV", _i32), ("HI", _i32), ("D", _i32),
        ("S", _i32), ("L", _i32),
        ("block_size", _i32), ("local_window", _i32),
        ("scale", ctypes.c_float),
        ("in_dtype", _i32), ("out_dtype", _i32),
    ]


class IndexArgs(ctypes.Structure):
    """Mirror of ``srswa_index_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_sh", _i64), ("q_sq", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("kbar_out", _vp), ("kb_sb", _i64), ("kb_sh", _i64), ("kb_sn", _i64),
        ("head_cls", _vp),
        ("q_pos", _vp), ("pos_sb", _i64), ("pos_sq", _i64),
        ("kv_len", _vp),
        ("scores", _vp), ("sc_sb", _i64), ("sc_sh", _i64), ("sc_sq", _i64),
        ("topk_idx", _vp), ("ti_sb", _i64), ("ti_sh", _i64), ("ti_sq", _i64),
        ("topk_val", _vp),
        ("B", _i32), ("HI", _i32), ("Lq", _i32), ("D", _i32), ("L", _i32), ("nblk", _i32),
        ("block_size", _i32), ("local_blocks", _i32), ("K", _i32), ("ascending", _i32),
        ("k_dtype", _i32),
    ]


class FwdArgs(ctypes.Structure):
    """Mirror of ``srswa_fwd_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64), ("q_sh", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("v", _vp), ("v_sb", _i64), ("v_st", _i64), ("v_sh", _i64),
        ("idx", _vp), ("idx_sb", _i64), ("idx_sh", _i64), ("idx_st", _i64),
        ("bias", _vp), ("bias_sb", _i64), ("bias_sh", _i64), ("bias_st", _i64),
        ("seg", _vp), ("seg_sb", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_st", _i64), ("o_sh", _i64),
        ("lse", _vp), ("lse_sb", _i64), ("lse_st", _i64), ("lse_sh", _i64),
        ("B", _i32), ("T", _i32), ("Sk", _i32), ("HQ", _i32), ("HKV", _i32), ("HI", _i32),
        ("D", _i32), ("S", _i32), ("block_size", _i32), ("local_window", _i32),
        ("scale", ctypes.c_float),
        ("dtype", _i32),
    ]


class PagedFwdArgs(ctypes.Structure):
    """Mirror of ``srswa_paged_fwd_args``."""

    _fields_ = [
        ("q", _vp), ("q_sn", _i64), ("q_sh", _i64),
        ("k_cache", _vp), ("k_sp", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("v_cache", _vp), ("v_sp", _i64), ("v_st", _i64), ("v_sh", _i64),
        ("topk", _vp), ("t_sh", _i64), ("t_sn", _i64),
        ("bias", _vp), ("b_sh", _i64), ("b_sn", _i64),
        ("block_table", _vp), ("bt_sr", _i64),
        ("cu_seqlens_q", _vp),
        ("seq_lens", _vp),
        ("prefix_lens", _vp),
        ("out", _vp), ("o_sn", _i64), ("o_sh", _i64),
        ("R", _i32), ("max_query_len", _i32), ("HQ", _i32), ("HKV", _i32), ("D", _i32), ("S", _i32),
        ("max_blocks", _i32), ("page_size", _i32), ("local_blocks", _i32),
        ("scale", ctypes.c_float),
        ("dtype", _i32),
        ("kv_fp8", _i32),
    ]


class BwdArgs(ctypes.Structure):
    """Mirror of ``srswa_bwd_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64), ("q_sh", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("v", _vp), ("v_sb", _i64), ("v_st", _i64), ("v_sh", _i64),
        ("o", _vp), ("o_sb", _i64), ("o_st", _i64), ("o_sh", _i64),
        ("lse", _vp), ("lse_sb", _i64), ("lse_st", _i64), ("lse_sh", _i64),
        ("dout", _vp), ("do_sb", _i64), ("do_st", _i64), ("do_sh", _i64),
        ("idx", _vp), ("idx_sb", _i64), ("idx_sh", _i64), ("idx_st", _i64),
        ("bias", _vp), ("bias_sb", _i64), ("bias_sh", _i64), ("bias_st", _i64),
        ("seg", _vp), ("seg_sb", _i64),
        ("dq", _vp), ("dq_sb", _i64), ("dq_st", _i64), ("dq_sh", _i64),
        ("dk", _vp), ("dk_sb", _i64), ("dk_st", _i64), ("dk_sh", _i64),
        ("dv", _vp), ("dv_sb", _i64), ("dv_st", _i64), ("dv_sh", _i64),
        ("dbias", _vp), ("db_sb", _i64), ("db_sh", _i64), ("db_st", _i64),
        ("B", _i32), ("T", _i32), ("Sk", _i32), ("HQ", _i32), ("HKV", _i32), ("HI", _i32),
        ("D", _i32), ("S", _i32), ("block_size", _i32), ("local_window", _i32),
        ("scale", ctypes.c_float),
        ("dtype", _i32),
    ]


class BlockMaxArgs(ctypes.Structure):
    """Mirror of ``srswa_blockmax_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_sc", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_sk", _i64),
        ("pos", _vp), ("pos_sb", _i64), ("pos_sc", _i64),
        ("seg", _vp), ("seg_sb", _i64), ("seg_sc", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_sc", _i64), ("o_sn", _i64),
        ("B", _i32), ("C", _i32), ("Sk", _i32), ("D", _i32), ("nblk", _i32), ("block_size", _i32),
        ("local_window", _i32),
        ("dtype", _i32),
    ]


class PagedDecodeArgs(ctypes.Structure):
    """Mirror of ``srswa_paged_decode_args``."""

    _fields_ = [
        ("q", _vp), ("q_sn", _i64), ("q_sh", _i64),
        ("k_cache", _vp), ("k_sp", _i64), ("k_st", _i64), ("k_sh", _i64),
        ("v_cache", _vp), ("v_sp", _i64), ("v_st", _i64), ("v_sh", _i64),
        ("topk", _vp), ("t_sh", _i64), ("t_sn", _i64), ("t_sk", _i64),
        ("bias", _vp),
        ("block_table", _vp), ("bt_sr", _i64),
        ("seq_lens", _vp),
        ("out", _vp), ("o_sn", _i64), ("o_sh", _i64),
        ("R", _i32), ("dql", _i32), ("HQ", _i32), ("HKV", _i32), ("D", _i32), ("topk_n", _i32),
        ("max_blocks", _i32), ("page_size", _i32), ("local_blocks", _i32),
        ("scale", ctypes.c_float),
        ("in_dtype", _i32), ("out_dtype", _i32),
        ("kv_fp8", _i32),
    ]


class KbarPagesArgs(ctypes.Structure):
    """Mirror of ``srswa_kbar_pages_args``."""

    _fields_ = [
        ("keys", _vp), ("k_sp", _i64), ("k_st", _i64),
        ("head_cls", _vp),
        ("block_table", _vp), ("bt_sr", _i64),
        ("seq_lens", _vp),
        ("kbar", _vp), ("kb_sp", _i64),
        ("R", _i32), ("max_blocks", _i32), ("page_size", _i32), ("D", _i32), ("tail_blocks", _i32),
        ("k_dtype", _i32),
    ]


class KbarScoresArgs(ctypes.Structure):
    """Mirror of ``srswa_kbar_scores_args``."""

    _fields_ = [
        ("q", _vp), ("q_sn", _i64),
        ("kbar", _vp), ("kb_sp", _i64),
        ("block_table", _vp), ("bt_sr", _i64),
        ("seq_lens", _vp),
        ("row_req", _vp),
        ("row_pos", _vp),
        ("cu_q", _vp),
        ("ctx", _vp),
        ("scores", _vp), ("sc_sn", _i64),
        ("nrows", _i32), ("R", _i32), ("dql", _i32), ("max_blocks", _i32), ("width", _i32),
        ("page_size", _i32), ("local_blocks", _i32), ("D", _i32), ("row_off", _i32),
    ]


class KbarPlanArgs(ctypes.Structure):
    """Mirror of ``srswa_kbar_plan_args``."""

    _fields_ = [
        ("keys", _vp), ("k_sp", _i64), ("k_st", _i64),
        ("head_cls", _vp),
        ("pages", _vp),
        ("tok", _vp),
        ("kbar", _vp), ("kb_sp", _i64),
        ("n", _i32), ("num_pages", _i32), ("page_size", _i32), ("D", _i32),
        ("k_dtype", _i32),
    ]


class RouteServeArgs(ctypes.Structure):
    """Mirror of ``srswa_route_serve_args``."""

    _fields_ = [
        ("scores", _vp), ("sc_sn", _i64),
        ("img", _vp), ("img_sn", _i64),
        ("out_idx", _vp), ("oi_sn", _i64),
        ("out_bias", _vp), ("ob_sn", _i64),
        ("rows", _i32), ("W", _i32), ("K", _i32), ("M", _i32),
        ("idx_scale", ctypes.c_float), ("prior_floor", ctypes.c_float), ("inv_sigma", ctypes.c_float),
    ]


class DashRouteTrainArgs(ctypes.Structure):
    """Mirror of ``srswa_dash_route_train_args``."""

    _fields_ = [
        ("scores", _vp), ("sc_sr", _i64),
        ("block_cand", _vp), ("bc_sr", _i64),
        ("img", _vp), ("img_sb", _i64),
        ("prior", _vp), ("p_sr", _i64),
        ("cand", _vp), ("c_sr", _i64),
        ("rows", _i32), ("nblk", _i32), ("rows_per_seq", _i32),
        ("scale", ctypes.c_float), ("neg", ctypes.c_float),
        ("dtype", _i32),
    ]


class DashRouteTrainBwdArgs(ctypes.Structure):
    """Mirror of ``srswa_dash_route_train_bwd_args``."""

    _fields_ = [
        ("d_prior", _vp), ("dp_sr", _i64),
        ("prior", _vp), ("p_sr", _i64),
        ("cand", _vp), ("c_sr", _i64),
        ("d_scores", _vp), ("ds_sr", _i64),
        ("rows", _i32), ("nblk", _i32),
        ("scale", ctypes.c_float),
        ("dtype", _i32),
    ]


class DashSelectTrainArgs(ctypes.Structure):
    """Mirror of ``srswa_dash_select_train_args``."""

    _fields_ = [
        ("prior", _vp), ("p_sr", _i64),
        ("cand", _vp), ("c_sr", _i64),
        ("topi", _vp), ("ti_sr", _i64),
        ("bias", _vp), ("b_sr", _i64),
        ("valid", _vp), ("v_sr", _i64),
        ("d_bias", _vp), ("db_sr", _i64),
        ("d_prior", _vp), ("dp_sr", _i64),
        ("rows", _i32), ("nblk", _i32), ("K", _i32),
        ("floor", ctypes.c_float), ("inv_sigma", ctypes.c_float),
        ("dtype", _i32),
    ]


class WinBoundsArgs(ctypes.Structure):
    """Mirror of ``srswa_win_bounds_args``."""

    _fields_ = [
        ("allow", _vp), ("a_sn", _i64),
        ("seq_lens", _vp),
        ("lo", _vp), ("hi", _vp),
        ("fit", _vp),
        ("rows", _i32), ("W", _i32), ("WQ", _i32), ("block_size", _i32), ("local_blocks", _i32),
        ("dql", _i32), ("tile", _i32),
    ]


class RouteArgs(ctypes.Structure):
    """Mirror of ``srswa_route_args``."""

    _fields_ = [
        ("scores", _vp), ("sc_sb", _i64), ("sc_sq", _i64),
        ("cand", _vp), ("cd_sb", _i64), ("cd_sq", _i64),
        ("topi", _vp), ("ti_sb", _i64), ("ti_sq", _i64),
        ("bias", _vp), ("bi_sb", _i64), ("bi_sq", _i64),
        ("valid", _vp), ("va_sb", _i64), ("va_sq", _i64),
        ("B", _i32), ("Lq", _i32), ("nblk", _i32), ("K", _i32), ("topm", _i32),
        ("idx_scale", ctypes.c_float), ("floor", ctypes.c_float),
        ("sigma", ctypes.c_double), ("mask_ids", _i32),
    ]


class PageStepArgs(ctypes.Structure):
    """Mirror of ``srswa_page_step_args``."""

    _fields_ = [
        ("input_ids", _vp), ("ids_i64", _i32),
        ("q_start", _vp), ("start_pos", _vp), ("gen_start", _vp),
        ("block_table", _vp), ("bt_i64", _i32), ("bt_sr", _i64),
        ("slot_mapping", _vp), ("slot_i64", _i32),
        ("s_page", _vp), ("s_mark", _vp), ("s_run", _vp), ("s_pp", _vp),
        ("q_page", _vp),
        ("image_token_id", _i64), ("page_token_id", _i64), ("num_decode_tokens", _i64),
        ("R", _i32), ("T", _i32), ("bt_w", _i32), ("n_slots", _i32), ("block_size", _i32), ("per_page", _i32),
        ("has_marker", _i32),
    ]


class CoordStepArgs(ctypes.Structure):
    """Mirror of ``srswa_coord_step_args``."""

    _fields_ = [
        ("input_ids", _vp), ("ids_i64", _i32),
        ("q_start", _vp), ("start_pos", _vp), ("gen_start", _vp), ("row", _vp),
        ("st_marker", _vp), ("st_pp", _vp), ("cnt", _vp), ("cnt_sr", _i64),
        ("tok", _vp), ("page", _vp), ("marker_out", _vp), ("pp_out", _vp),
        ("image_token_id", _i64), ("page_token_id", _i64), ("num_decode_tokens", _i64),
        ("R", _i32), ("T", _i32), ("n_rows", _i32), ("pages", _i32), ("has_marker", _i32),
    ]


class PageIdsArgs(ctypes.Structure):
    """Mirror of ``srswa_page_ids_args``."""

    _fields_ = [
        ("ids", _vp), ("ids_i64", _i32), ("id_sb", _i64),
        ("img_mask", _vp), ("img_page", _vp), ("q_page", _vp), ("o_sb", _i64),
        ("row_counts", _vp),
        ("image_token_id", _i64), ("page_token_id", _i64),
        ("B", _i32), ("L", _i32), ("n_ids", _i32), ("per_page", _i32), ("page_scope_prefill", _i32),
    ]


class PagePosArgs(ctypes.Structure):
    """Mirror of ``srswa_page_pos_args``."""

    _fields_ = [
        ("ids", _vp), ("ids_i64", _i32), ("id_sb", _i64),
        ("page", _vp), ("prefill", _vp), ("o_sb", _i64),
        ("row_info", _vp),
        ("tok", _vp),
        ("pf_cnt", _vp), ("pf_sb", _i64),
        ("image_token_id", _i64), ("page_token_id", _i64),
        ("B", _i32), ("L", _i32), ("n_ids", _i32), ("n_pg", _i32),
    ]


class PageMetaArgs(ctypes.Structure):
    """Mirror of ``srswa_page_meta_args``."""

    _fields_ = [
        ("input_ids", _vp), ("ids_i64", _i32),
        ("block_table", _vp), ("bt_i64", _i32), ("bt_sr", _i64),
        ("seq_lens", _vp), ("seq_i64", _i32),
        ("slot_mapping", _vp), ("slot_i64", _i32),
        ("coord_row", _vp),
        ("s_page", _vp), ("s_mark", _vp), ("s_run", _vp), ("s_pp", _vp),
        ("c_mark", _vp), ("c_pp", _vp), ("c_cnt", _vp), ("cnt_sr", _i64),
        ("q_page", _vp), ("tok", _vp), ("page", _vp),
        ("image_token_id", _i64), ("page_token_id", _i64),
        ("R", _i32), ("bt_w", _i32), ("n_slots", _i32), ("n_rows", _i32), ("max_pages", _i32),
        ("block_size", _i32), ("per_page", _i32), ("has_marker", _i32),
    ]


class PageAllowArgs(ctypes.Structure):
    """Mirror of ``srswa_page_allow_args``."""

    _fields_ = [
        ("block_table", _vp), ("bt_i64", _i32), ("bt_sr", _i64),
        ("s_page", _vp), ("n_slots", _i64),
        ("q_page", _vp),
        ("seq_lens", _vp), ("seq_i64", _i32),
        ("out", _vp), ("out_sr", _i64),
        ("R", _i32), ("bt_w", _i32), ("max_block", _i32), ("num_blocks", _i32), ("block_size", _i32),
    ]


class LocalUnionArgs(ctypes.Structure):
    """Mirror of ``srswa_local_union_args``."""

    _fields_ = [
        ("allow", _vp), ("a_sr", _i64),
        ("out", _vp), ("o_sr", _i64),
        ("seq_lens", _vp), ("seq_i64", _i32),
        ("R", _i32), ("a_w", _i32), ("o_w", _i32), ("max_block", _i32), ("block_size", _i32),
        ("local_blocks", _i32),
    ]


class CosSinArgs(ctypes.Structure):
    """Mirror of ``srswa_cos_sin_args``."""

    _fields_ = [
        ("tok", _vp), ("tok_i64", _i32),
        ("page", _vp), ("page_i64", _i32),
        ("inv_tok", _vp), ("inv_page", _vp),
        ("cos", _vp), ("c_st", _i64),
        ("sin", _vp), ("s_st", _i64),
        ("page_mod", _i64),
        ("T", _i32), ("dim", _i32), ("n_tok", _i32), ("out_dtype", _i32),
    ]


class RopeArgs(ctypes.Structure):
    """Mirror of ``srswa_rope_args``."""

    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_ss", _i64), ("x_sh", _i64),
        ("ox", _vp), ("ox_sb", _i64), ("ox_ss", _i64), ("ox_sh", _i64),
        ("y", _vp), ("y_sb", _i64), ("y_ss", _i64), ("y_sh", _i64),
        ("oy", _vp), ("oy_sb", _i64), ("oy_ss", _i64), ("oy_sh", _i64),
        ("cos", _vp), ("c_sb", _i64), ("c_ss", _i64),
        ("sin", _vp), ("s_sb", _i64), ("s_ss", _i64),
        ("B", _i32), ("S", _i32), ("HX", _i32), ("HY", _i32), ("head_dim", _i32), ("dtype", _i32),
    ]


class BlockBoundsArgs(ctypes.Structure):
    """Mirror of ``srswa_block_bounds_args``."""

    _fields_ = [
        ("ids", _vp), ("ids_i64", _i32), ("id_sb", _i64),
        ("bounds", _vp), ("bd_sb", _i64),
        ("B", _i32), ("L", _i32), ("nblk", _i32), ("block_size", _i32),
    ]


class CandidateArgs(ctypes.Structure):
    """Mirror of ``srswa_candidate_args``."""

    _fields_ = [
        ("bounds", _vp), ("bd_sb", _i64),
        ("ids", _vp), ("ids_i64", _i32), ("id_sb", _i64),
        ("qpage", _vp), ("qp_i64", _i32), ("qp_sb", _i64),
        ("pos", _vp), ("pos_i64", _i32), ("pos_sb", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_sq", _i64),
        ("B", _i32), ("nq", _i32), ("qlen", _i32), ("L", _i32), ("nblk", _i32), ("nbd", _i32),
        ("block_size", _i32), ("range_test", _i32),
    ]


class KlArgs(ctypes.Structure):
    """Mirror of ``srswa_kl_args``."""

    _fields_ = [
        ("q_idx", _vp), ("qi_sb", _i64), ("qi_sh", _i64), ("qi_st", _i64),
        ("idx_k", _vp), ("ik_sb", _i64), ("ik_st", _i64),
        ("q_main", _vp), ("qm_sb", _i64), ("qm_sh", _i64), ("qm_st", _i64),
        ("k_main", _vp), ("km_sb", _i64), ("km_sh", _i64), ("km_st", _i64),
        ("sel", _vp), ("sel_sb", _i64), ("sel_sh", _i64), ("sel_st", _i64),
        ("pos", _vp), ("pos_sb", _i64),
        ("seg", _vp), ("seg_sb", _i64),
        ("kl", _vp), ("kl_sb", _i64), ("kl_sh", _i64),
        ("valid", _vp), ("va_sb", _i64), ("va_sh", _i64),
        ("dsel", _vp), ("ds_sb", _i64), ("ds_sh", _i64), ("ds_st", _i64),
        ("B", _i32), ("HI", _i32), ("HQ", _i32), ("HKV", _i32), ("T", _i32), ("Sk", _i32), ("D", _i32),
        ("K", _i32), ("block_size", _i32), ("local_window", _i32),
        ("scaling", ctypes.c_float),
        ("dtype", _i32),
        ("slots_are_blocks", _i32),
        ("side_stream", _vp), ("fork_event", _vp), ("join_event", _vp),
    ]


class KlBwdArgs(ctypes.Structure):
    """Mirror of ``srswa_kl_bwd_args``."""

    _fields_ = [
        ("q_idx", _vp), ("qi_sb", _i64), ("qi_sh", _i64), ("qi_st", _i64),
        ("idx_k", _vp), ("ik_sb", _i64), ("ik_st", _i64),
        ("sel", _vp), ("sel_sb", _i64), ("sel_sh", _i64), ("sel_st", _i64),
        ("dsel", _vp), ("ds_sb", _i64), ("ds_sh", _i64), ("ds_st", _i64),
        ("grad", _vp), ("g_sb", _i64), ("g_sh", _i64),
        ("dq_idx", _vp), ("dq_sb", _i64), ("dq_sh", _i64), ("dq_st", _i64),
        ("dk_idx", _vp), ("dk_sb", _i64), ("dk_st", _i64),
        ("B", _i32), ("HI", _i32), ("T", _i32), ("Sk", _i32), ("D", _i32), ("K", _i32), ("block_size", _i32),
        ("dtype", _i32),
        ("slots_are_blocks", _i32),
        ("side_stream", _vp), ("fork_event", _vp), ("join_event", _vp),
    ]


class HcScoreArgs(ctypes.Structure):
    """Mirror of ``srswa_hc_score_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64),
        ("head_cls", _vp),
        ("pos", _vp), ("pos_sb", _i64), ("pos_st", _i64),
        ("kbar", _vp), ("kb_sb", _i64),
        ("z", _vp), ("z_sb", _i64), ("z_st", _i64),
        ("B", _i32), ("S", _i32), ("D", _i32), ("nblk", _i32), ("block_size", _i32), ("local_blocks", _i32),
    ]


class HcScoreBwdArgs(ctypes.Structure):
    """Mirror of ``srswa_hc_score_bwd_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64),
        ("head_cls", _vp),
        ("pos", _vp), ("pos_sb", _i64), ("pos_st", _i64),
        ("kbar", _vp), ("kb_sb", _i64),
        ("z", _vp), ("z_sb", _i64), ("z_st", _i64),
        ("gz", _vp), ("gz_sb", _i64), ("gz_st", _i64),
        ("dq", _vp), ("dq_sb", _i64), ("dq_st", _i64),
        ("dk", _vp), ("dk_sb", _i64), ("dk_st", _i64),
        ("dhc", _vp),
        ("B", _i32), ("S", _i32), ("D", _i32), ("nblk", _i32), ("block_size", _i32), ("local_blocks", _i32),
    ]


class BmScoreArgs(ctypes.Structure):
    """Mirror of ``srswa_bm_score_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64),
        ("pos", _vp), ("pos_sb", _i64), ("pos_st", _i64),
        ("z", _vp), ("z_sb", _i64), ("z_st", _i64),
        ("code", _vp),
        ("tiemask", _vp),
        ("B", _i32), ("S", _i32), ("D", _i32), ("nblk", _i32), ("block_size", _i32), ("local_window", _i32),
    ]


class BmScoreBwdArgs(ctypes.Structure):
    """Mirror of ``srswa_bm_score_bwd_args``."""

    _fields_ = [
        ("q", _vp), ("q_sb", _i64), ("q_st", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_st", _i64),
        ("pos", _vp), ("pos_sb", _i64), ("pos_st", _i64),
        ("code", _vp),
        ("tiemask", _vp),
        ("gz", _vp), ("gz_sb", _i64), ("gz_st", _i64),
        ("dq", _vp), ("dq_sb", _i64), ("dq_st", _i64),
        ("dk", _vp), ("dk_sb", _i64), ("dk_st", _i64),
        ("B", _i32), ("S", _i32), ("D", _i32), ("nblk", _i32), ("block_size", _i32), ("local_window", _i32),
    ]


# name -> (restype, argtypes) of every exported entry point
SIGNATURES = {
    "srswa_version": (ctypes.c_int, []),
    "srswa_last_error": (ctypes.c_char_p, []),
    "srswa_gather_decode_workspace": (ctypes.c_size_t, [ctypes.POINTER(DecodeArgs)]),
    "srswa_gather_decode": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_gather_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp]),
    "srswa_index_workspace": (ctypes.c_size_t, [ctypes.POINTER(IndexArgs)]),
    "srswa_index_meanpool_topk": (ctypes.c_int, [ctypes.POINTER(IndexArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_topk_rows": (ctypes.c_int, [_vp, _i64, _i32, _i64, _i32, _i32, ctypes.c_float, _vp, _vp,
                                       _i64, _vp]),
    "srswa_gather_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), _vp]),
    "srswa_gather_fwd_workspace": (ctypes.c_size_t, [ctypes.POINTER(FwdArgs)]),
    "srswa_gather_fwd_ws": (ctypes.c_int, [ctypes.POINTER(FwdArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_gather_fwd_paged": (ctypes.c_int, [ctypes.POINTER(PagedFwdArgs), _vp]),
    "srswa_gather_bwd_workspace": (ctypes.c_size_t, [ctypes.POINTER(BwdArgs)]),
    "srswa_gather_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_block_max_score": (ctypes.c_int, [ctypes.POINTER(BlockMaxArgs), _vp]),
    "srswa_dash_route": (ctypes.c_int, [ctypes.POINTER(RouteArgs), _vp]),
    "srswa_kbar_pages": (ctypes.c_int, [ctypes.POINTER(KbarPagesArgs), _vp]),
    "srswa_kbar_scores": (ctypes.c_int, [ctypes.POINTER(KbarScoresArgs), _vp]),
    "srswa_kbar_plan": (ctypes.c_int, [ctypes.POINTER(KbarPlanArgs), _vp]),
    "srswa_route_serve": (ctypes.c_int, [ctypes.POINTER(RouteServeArgs), _vp]),
    "srswa_win_bounds": (ctypes.c_int, [ctypes.POINTER(WinBoundsArgs), _vp]),
    "srswa_dash_route_train": (ctypes.c_int, [ctypes.POINTER(DashRouteTrainArgs), _vp]),
    "srswa_dash_route_train_bwd": (ctypes.c_int, [ctypes.POINTER(DashRouteTrainBwdArgs), _vp]),
    "srswa_dash_select_train": (ctypes.c_int, [ctypes.POINTER(DashSelectTrainArgs), _vp]),
    "srswa_dash_select_train_bwd": (ctypes.c_int, [ctypes.POINTER(DashSelectTrainArgs), _vp]),
    "srswa_gather_decode_paged_workspace": (ctypes.c_size_t, [ctypes.POINTER(PagedDecodeArgs)]),
    "srswa_gather_decode_paged": (ctypes.c_int, [ctypes.POINTER(PagedDecodeArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_page_decode_meta": (ctypes.c_int, [ctypes.POINTER(PageMetaArgs), _vp]),
    "srswa_page_step": (ctypes.c_int, [ctypes.POINTER(PageStepArgs), _vp]),
    "srswa_coord_step": (ctypes.c_int, [ctypes.POINTER(CoordStepArgs), _vp]),
    "srswa_page_ids": (ctypes.c_int, [ctypes.POINTER(PageIdsArgs), _vp]),
    "srswa_page_rope_pos": (ctypes.c_int, [ctypes.POINTER(PagePosArgs), _vp]),
    "srswa_page_rope_tok": (ctypes.c_int, [ctypes.POINTER(PagePosArgs), _vp]),
    "srswa_page_decode_allow_workspace": (ctypes.c_int, [ctypes.POINTER(PageAllowArgs), _szp]),
    "srswa_page_decode_allow": (ctypes.c_int, [ctypes.POINTER(PageAllowArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_page_local_union": (ctypes.c_int, [ctypes.POINTER(LocalUnionArgs), _vp]),
    "srswa_page2d_cos_sin": (ctypes.c_int, [ctypes.POINTER(CosSinArgs), _vp]),
    "srswa_page2d_rope": (ctypes.c_int, [ctypes.POINTER(RopeArgs), _vp]),
    "srswa_page_block_bounds": (ctypes.c_int, [ctypes.POINTER(BlockBoundsArgs), _vp]),
    "srswa_page_candidate_mask": (ctypes.c_int, [ctypes.POINTER(CandidateArgs), _vp]),
    "srswa_gather_kl_fwd": (ctypes.c_int, [ctypes.POINTER(KlArgs), _vp]),
    "srswa_gather_kl_fwd_workspace": (ctypes.c_size_t, [ctypes.POINTER(KlArgs)]),
    "srswa_gather_kl_fwd_ws": (ctypes.c_int, [ctypes.POINTER(KlArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_gather_kl_bwd_workspace": (ctypes.c_int, [ctypes.POINTER(KlBwdArgs), _szp]),
    "srswa_gather_kl_bwd": (ctypes.c_int, [ctypes.POINTER(KlBwdArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_hc_score_fwd": (ctypes.c_int, [ctypes.POINTER(HcScoreArgs), _vp]),
    "srswa_hc_score_bwd_workspace": (ctypes.c_int, [ctypes.POINTER(HcScoreBwdArgs), _szp]),
    "srswa_hc_score_bwd": (ctypes.c_int, [ctypes.POINTER(HcScoreBwdArgs), _vp, ctypes.c_size_t, _vp]),
    "srswa_bm_score_fwd": (ctypes.c_int, [ctypes.POINTER(BmScoreArgs), _vp]),
    "srswa_bm_score_bwd_workspace": (ctypes.c_int, [ctypes.POINTER(BmScoreBwdArgs), _szp]),
    "srswa_bm_score_bwd": (ctypes.c_int, [ctypes.POINTER(BmScoreBwdArgs), _vp, ctypes.c_size_t, _vp]),
}

STRUCTS = {"srswa_decode_args": DecodeArgs, "srswa_index_args": IndexArgs,
           "srswa_fwd_args": FwdArgs, "srswa_paged_fwd_args": PagedFwdArgs, "srswa_bwd_args": BwdArgs,
           "srswa_blockmax_args": BlockMaxArgs, "srswa_route_args": RouteArgs,
           "srswa_paged_decode_args": PagedDecodeArgs, "srswa_kbar_pages_args": KbarPagesArgs,
           "srswa_kbar_scores_args": KbarScoresArgs, "srswa_kbar_plan_args": KbarPlanArgs,
           "srswa_route_serve_args": RouteServeArgs, "srswa_win_bounds_args": WinBoundsArgs,
           "srswa_dash_route_train_args": DashRouteTrainArgs,
           "srswa_dash_route_train_bwd_args": DashRouteTrainBwdArgs,
           "srswa_dash_select_train_args": DashSelectTrainArgs,
           "srswa_page_meta_args": PageMetaArgs, "srswa_page_step_args": PageStepArgs,
           "srswa_coord_step_args": CoordStepArgs, "srswa_page_ids_args": PageIdsArgs,
           "srswa_page_pos_args": PagePosArgs,
           "srswa_page_allow_args": PageAllowArgs, "srswa_local_union_args": LocalUnionArgs,
           "srswa_cos_sin_args": CosSinArgs, "srswa_rope_args": RopeArgs,
           "srswa_block_bounds_args": BlockBoundsArgs, "srswa_candidate_args": CandidateArgs,
           "srswa_kl_args": KlArgs, "srswa_kl_bwd_args": KlBwdArgs,
           "srswa_hc_score_args": HcScoreArgs, "srswa_hc_score_bwd_args": HcScoreBwdArgs,
           "srswa_bm_score_args": BmScoreArgs, "srswa_bm_score_bwd_args": BmScoreBwdArgs}

_lib = None
_lock = threading.Lock()


class UnsupportedShape(Exception):
    """The kernels do not cover this shape/dtype (reference contract: caller falls back)."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libsrswa.so not built ({LIB_PATH}); run "
                    "`python unlimited-ocr_amd/build.py` (hipcc, gfx950)")
            l = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(l, name)
                fn.restype = res
                fn.argtypes = args
            _lib = l
    return _lib


def check(status: int, what: str) -> None:
    if status == SRSWA_OK:
        return
    msg = lib().srswa_last_error().decode(errors="replace")
    if status == SRSWA_UNSUPPORTED:
        raise UnsupportedShape(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed (status {status}): {msg}")


FP8_CODES = {}
for _name, _code in (("float8_e4m3fn", 3), ("float8_e4m3fnuz", 4), ("float8_e5m2", 5), ("float8_e5m2fnuz", 6)):
    if hasattr(torch, _name):
        FP8_CODES[getattr(torch, _name)] = _code


def fp8_code(dt: torch.dtype) -> int:
    """srswa_dtype of an fp8 K/V cache dtype, 0 for any other dtype."""
    return FP8_CODES.get(dt, 0)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return SRSWA_F32
    if dt == torch.bfloat16:
        return SRSWA_BF16
    if dt == torch.float16:
        return SRSWA_F16
    raise UnsupportedShape(f"dtype {dt} not supported")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_scratch_cache: dict = {}


def _stream_key(device: torch.device):
    return (device.index, torch.cuda.current_stream(device).cuda_stream)


def scratch(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Device scratch (no content requirement), cached per (device, stream)."""
    if nbytes <= 0:
        return None
    key = _stream_key(device)
    buf = _scratch_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _scratch_cache[key] = buf
    return buf
