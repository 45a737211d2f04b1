"""ctypes binding of liblogkv_hip.so (the C ABI in include/logkv_hip.h).

The library is the only compute path: if it is missing or a call fails, this
module raises; nothing falls back to a CPU or PyTorch implementation.
"""

from __future__ import annotations

import ctypes as C
from functools import lru_cache
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblogkv_hip.so"

LOGKV_OK, LOGKV_EINVAL, LOGKV_ERUNTIME = 0, 1, 2

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32


class LadderView(C.Structure):
    _fields_ = [
        ("level_k", _p), ("level_v", _p), ("level_w", _p), ("level_p_lo", _p), ("level_p_hi", _p),
        ("level_sum_wp", _p), ("level_order", _p), ("pad_mask", _p), ("level_count", _p),
        ("centroid", _p), ("n_eff", _p), ("n_total", _p), ("p_hi_c", _p), ("level0_phase", _p),
        ("alive", _p), ("s_h", _p),
        ("n_batch", _i32), ("n_groups", _i32), ("k_max", _i32), ("levels", _i32), ("slots", _i32),
        ("dk", _i32), ("dv", _i32),
    ]


class RowsView(C.Structure):
    _fields_ = [
        ("k", _p), ("k_sb", _i64), ("k_sg", _i64), ("k_st", _i64),
        ("v", _p), ("v_sb", _i64), ("v_sg", _i64), ("v_st", _i64),
        ("pos", _p), ("pos_sb", _i64), ("counts", _p), ("tokens", _i32),
    ]


class RouteParams(C.Structure):
    _fields_ = [("eta", C.c_float), ("g0", C.c_float), ("lam", C.c_float),
                ("late_joins", _i32), ("beta_merge", _i32), ("center_tile", _i32), ("hard_cap", C.c_float),
                ("hard_cap_rows", _i32), ("merge_passes", _i32)]


class RecentArgs(C.Structure):
    _fields_ = [("recent_k", _p), ("recent_k_raw", _p), ("recent_v", _p), ("recent_pos", _p), ("recent_ends", _p),
                ("n_batch", _i32), ("n_groups", _i32), ("cap", _i32), ("dk", _i32), ("dkr", _i32), ("dv", _i32),
                ("k", _p), ("k_sb", _i64), ("k_sg", _i64), ("k_st", _i64),
                ("k_raw", _p), ("kr_sb", _i64), ("kr_sg", _i64), ("kr_st", _i64),
                ("v", _p), ("v_sb", _i64), ("v_sg", _i64), ("v_st", _i64),
                ("pos", _p), ("pos_sb", _i64), ("pos_st", _i64), ("ends", _p), ("ends_sb", _i64)]


class SpanArgs(C.Structure):
    _fields_ = [
        ("pool_k", _p), ("pk_sb", _i64), ("pk_sg", _i64), ("pk_st", _i64),
        ("pool_v", _p), ("pv_sb", _i64), ("pv_sg", _i64), ("pv_st", _i64),
        ("flush_k", _p), ("fk_sb", _i64), ("fk_sg", _i64), ("fk_st", _i64),
        ("flush_v", _p), ("fv_sb", _i64), ("fv_sg", _i64), ("fv_st", _i64),
        ("old_width", _i32), ("tokens", _p), ("span_offsets", _p), ("span_rows", _p), ("n_spans", _i32),
        ("n_groups", _i32), ("dk", _i32), ("dv", _i32),
        ("centroids", _p), ("centroid_valid", _p), ("k_max", _i32), ("beta_novelty", _i32),
        ("n_spans_dev", _p),
    ]


class AlphaSelectArgs(C.Structure):
    _fields_ = [
        ("span_len", _p), ("span_closed", _p), ("span_count", _p), ("pool_pos", _p),
        ("new_pos", _p), ("np_sb", _i64), ("ends", _p), ("ends_sb", _i64), ("tokens", _i32),
        ("n_batch", _i32), ("budget", _i32), ("max_span", _i32), ("rows", SpanArgs),
        ("keep", _p), ("archive", _p), ("archive_count", _p), ("new_span_len", _p), ("new_span_closed", _p),
        ("new_span_count", _p), ("alpha_count", _p), ("scores", _p), ("count_rows", _i32),
    ]


class PartitionArgs(C.Structure):
    _fields_ = [
        ("pool_k", _p), ("pk_sb", _i64), ("pk_sg", _i64), ("pk_st", _i64),
        ("pool_v", _p), ("pv_sb", _i64), ("pv_sg", _i64), ("pv_st", _i64),
        ("pool_pos", _p), ("pp_sb", _i64),
        ("flush_k", _p), ("fk_sb", _i64), ("fk_sg", _i64), ("fk_st", _i64),
        ("flush_v", _p), ("fv_sb", _i64), ("fv_sg", _i64), ("fv_st", _i64),
        ("flush_pos", _p), ("fp_sb", _i64),
        ("old_width", _i32), ("keep", _p), ("archive", _p),
        ("P", _i32), ("A", _i32), ("n_batch", _i32), ("n_groups", _i32), ("dk", _i32), ("dv", _i32),
        ("out_pool_k", _p), ("out_pool_v", _p), ("out_pool_pos", _p), ("out_pool_valid", _p),
        ("arch_k", _p), ("arch_v", _p), ("arch_pos", _p),
    ]


class ReadoutView(C.Structure):
    _fields_ = [
        ("level_k", _p), ("level_v", _p), ("level_w", _p), ("level_sum_wp", _p), ("level_count", _p),
        ("n_batch", _i32), ("n_groups", _i32), ("k_max", _i32), ("levels", _i32), ("slots", _i32),
        ("dk", _i32), ("dv", _i32),
        ("alpha_k", _p), ("alpha_v", _p), ("alpha_pos", _p), ("alpha_valid", _p),
        ("alpha_cap", _i32), ("alpha_count", _i32),
        ("recent_k", _p), ("recent_v", _p), ("recent_cap", _i32), ("recent_count", _i32),
        ("cos", _p), ("sin", _p), ("cos_s0", _i64), ("cos_s1", _i64), ("sin_s0", _i64), ("sin_s1", _i64),
        ("rope_n", _i32), ("table_bf16", _i32), ("rope_rows", _i64), ("alpha_count_dev", _p),
    ]


class PackArgs(C.Structure):
    _fields_ = [
        ("cur_k", _p), ("ck_sb", _i64), ("ck_sg", _i64), ("ck_st", _i64),
        ("cur_v", _p), ("cv_sb", _i64), ("cv_sg", _i64), ("cv_st", _i64),
        ("cur_len", _i32), ("out_k", _p), ("out_v", _p), ("out_cap", _i32), ("dim", _i32),
        ("skip_pooled", _i32), ("recent_start", _i32), ("out_w", _p), ("out_valid", _p),
    ]


class SlotPackArgs(C.Structure):
    _fields_ = [
        ("k", _p), ("k_sb", _i64), ("k_sg", _i64), ("k_st", _i64),
        ("v", _p), ("v_sb", _i64), ("v_sg", _i64), ("v_st", _i64),
        ("w", _p), ("w_sb", _i64), ("w_sg", _i64),
        ("m", _p), ("m_sb", _i64), ("m_sg", _i64), ("s_m", _i32),
        ("valid", _p), ("valid_sb", _i64), ("valid_sg", _i64), ("s_valid", _i32),
        ("lam", C.c_float),
        ("n_batch", _i32), ("n_groups", _i32), ("slots", _i32), ("dk", _i32), ("dv", _i32), ("dim", _i32),
        ("out_cap", _i32), ("out_k", _p), ("out_v", _p),
    ]


class AttentionArgs(C.Structure):
    _fields_ = [
        ("q", _p), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64),
        ("n_batch", _i32), ("n_heads", _i32), ("n_groups", _i32), ("tq", _i32), ("dk", _i32), ("dv", _i32),
        ("dim", _i32), ("k", _p), ("v", _p), ("cap", _i32), ("tail", _i32), ("causal_tail", _i32),
        ("scale", C.c_float), ("inv_scale_bf16", C.c_float),
        ("out", _p), ("o_sb", _i64), ("o_sh", _i64), ("o_st", _i64), ("alpha_count_dev", _p),
    ]


class BetaArgs(C.Structure):
    _fields_ = [
        ("k", _p), ("k_st", _i64), ("k_f32", _i32), ("v", _p), ("v_st", _i64), ("v_f32", _i32),
        ("w", _p), ("p_lo", _p), ("p_hi", _p), ("sum_wp", _p), ("order", _p), ("pad", _p),
        ("n_rows", _i64), ("dk", _i32), ("dv", _i32), ("layout", _p), ("n_groups", _i64), ("cuts", _p),
        ("apply", _i32), ("out_k", _p), ("out_v", _p), ("out_w", _p), ("out_p_lo", _p), ("out_p_hi", _p),
        ("out_sum_wp", _p), ("out_order", _p), ("out_pad", _p),
    ]


class AttentionGradArgs(C.Structure):
    _fields_ = [
        ("dout", _p), ("do_sb", _i64), ("do_sh", _i64), ("do_st", _i64),
        ("dq", _p), ("dq_sb", _i64), ("dq_sh", _i64), ("dq_st", _i64),
        ("dk", _p), ("dv", _p), ("grad_rows", _i32),
    ]


class OpLogView(C.Structure):
    _fields_ = [("rows", _p), ("lengths", _p), ("capacity", _i64)]


# Op codes of the route op-log (litgpt/log_kv_cache.py:90-94).
OP_NEW_CLUSTER, OP_NEW_SEGMENT, OP_JOIN, OP_WARD_MERGE, OP_PAD_INSERT = 0, 1, 2, 3, 4

# Replay status bits of logkv_replay_commit -> what failed.
REPLAY_ERRORS = {
    1: "a log row is not a NEW_CLUSTER / JOIN of segment 0 of a cluster in range (segment pads are not recorded "
       "on this path; Ward merges only lead a unified-routed flush's rows, between two live clusters)",
    2: "a logged position is not in the current flush positions",
    4: "the current flush positions contain duplicate token ids",
    8: "the log holds fewer rows than the flush has tokens",
    16: "a flush token is not consumed exactly once by the log",
    32: "a NEW_CLUSTER names a live cluster or a JOIN names a dead one",
    64: "a cluster's logged rows are not in increasing position order",
}

# Exported symbol -> (restype, argtypes); the tests check this table against the header.
SIGNATURES = {
    "logkv_last_error": (C.c_char_p, []),
    "logkv_route_workspace_bytes": (_i64, [C.POINTER(LadderView), _i32, _i32]),
    "logkv_attach_assign": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams),
                                   _p, _i64, _p, _p, _p]),
    "logkv_route_commit": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams),
                                  _p, _i64, _p, _p, _p]),
    "logkv_commit_only": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams),
                                 _p, _i64, _p, _p, _p]),
    "logkv_unified_workspace_bytes": (_i64, [C.POINTER(LadderView), _i32, _i32]),
    "logkv_unified_stats_offset": (_i64, [C.POINTER(LadderView), _i32, _i32]),
    "logkv_unified_plan": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams), _p, _p, _i64,
                                  _p, _p]),
    "logkv_unified_commit": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams), _p, _i64,
                                    _i32, _p]),
    "logkv_record_ops": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), _p, _i64, C.POINTER(OpLogView), _p]),
    "logkv_unified_record_ops": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams), _p, _i64,
                                        C.POINTER(OpLogView), _p]),
    "logkv_unified_replay_plan": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams), _p,
                                         _i64, C.POINTER(OpLogView), _p, _p, _p, _p]),
    "logkv_unified_decisions": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams), _p, _i64,
                                       _p, _p, _p, _p, _i32, _p]),
    "logkv_replay_commit": (_i32, [C.POINTER(LadderView), C.POINTER(RowsView), C.POINTER(RouteParams),
                                   _p, _i64, C.POINTER(OpLogView), _i64, _p, _p]),
    "logkv_score_spans": (_i32, [C.POINTER(SpanArgs), _p, _p]),
    "logkv_alpha_partition": (_i32, [C.POINTER(PartitionArgs), _p]),
    "logkv_alpha_select_workspace_bytes": (_i64, [C.POINTER(AlphaSelectArgs)]),
    "logkv_alpha_select": (_i32, [C.POINTER(AlphaSelectArgs), _p, _i64, _p]),
    "logkv_plan_table_ints": (_i64, [C.POINTER(ReadoutView)]),
    "logkv_mid_plan": (_i32, [C.POINTER(ReadoutView), _p, _p]),
    "logkv_pack": (_i32, [C.POINTER(ReadoutView), C.POINTER(PackArgs), _p, _p]),
    "logkv_pack_slots": (_i32, [C.POINTER(SlotPackArgs), _p]),
    "logkv_attention_workspace_bytes": (_i64, [C.POINTER(AttentionArgs)]),
    "logkv_decode_attention": (_i32, [C.POINTER(AttentionArgs), _p, _i64, _p, _i64, _p]),
    "logkv_decode_attention_static": (_i32, [C.POINTER(AttentionArgs), _p, _i64, _p]),
    "logkv_beta_merge": (_i32, [C.POINTER(BetaArgs), _p, _p]),
    "logkv_chunk_backward_workspace_bytes": (_i64, [C.POINTER(AttentionArgs)]),
    "logkv_chunk_attention_backward": (_i32, [C.POINTER(AttentionArgs), _p, _i64, C.POINTER(AttentionGradArgs), _p,
                                              _i64, _p]),
    "logkv_chunk_workspace_bytes": (_i64, [C.POINTER(AttentionArgs)]),
    "logkv_recent_append": (_i32, [C.POINTER(RecentArgs), _i32, _i32, _p]),
    "logkv_recent_shift": (_i32, [C.POINTER(RecentArgs), _i32, _i32, _p]),
    "logkv_chunk_attention": (_i32, [C.POINTER(AttentionArgs), _p, _i64, _p, _i64, _p]),
}


class LogKVError(RuntimeError):
    pass


@lru_cache(maxsize=1)
def lib() -> C.CDLL:
    if not LIB_PATH.exists():
        raise LogKVError(f"{LIB_PATH} is not built; run `python __graft_entry__.py` or logkv_amd/build.py")
    handle = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = res, args
    return handle


def check(rc: int, what: str) -> None:
    if rc == LOGKV_OK:
        return
    msg = lib().logkv_last_error().decode(errors="replace")
    if rc == LOGKV_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise LogKVError(f"{what}: {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must live on a ROCm device (got {t.device}); the LogKV HIP library has no CPU path")


# Activation dtypes the cache accepts. Its entries are always stored as bfloat16 (the kernels read and
# write bf16 rows with fp32 arithmetic); rows of another activation dtype are rounded to bf16 (nearest
# even) where they enter, and readouts are returned in the caller's dtype.
ACTIVATION_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def check_activation_dtype(dtype: torch.dtype) -> None:
    if dtype not in ACTIVATION_DTYPES:
        raise NotImplementedError(f"logkv_amd takes bfloat16, float16 or float32 activations, not {dtype}")


def as_storage(t):
    """``t`` at the cache's storage precision: bf16 tensors (and None) pass through, float16 / float32
    rows are rounded to bf16 by a differentiable cast."""
    if t is None or not isinstance(t, torch.Tensor) or t.dtype == torch.bfloat16:
        return t
    check_activation_dtype(t.dtype)
    return t.to(torch.bfloat16)
