"""ctypes binding of libmtpx.so (the C ABI declared in include/mtpx.h).

The library is required: there is no fallback path.  A missing or unloadable
libmtpx.so raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmtpx.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "mtpx.h")

P = C.c_void_p
I32, I64, U32, U64, F32 = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float
INT = C.c_int


class Handle(C.Structure):
    _fields_ = [("ctx", P)]


class MoEWeights(C.Structure):
    _fields_ = [("hidden", INT), ("experts", INT), ("top_k", INT), ("expert_width", INT),
                ("group_size", INT)] + [(n, P) for n in (
                    "router", "shared_gate",
                    "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
                    "sh_gate_w", "sh_gate_s", "sh_gate_b", "sh_up_w", "sh_up_s", "sh_up_b",
                    "sh_down_w", "sh_down_s", "sh_down_b",
                    "gate_sb", "up_sb", "down_sb", "sh_gate_sb", "sh_up_sb", "sh_down_sb",
                    "shared_gate_w", "shared_gate_s", "shared_gate_b", "shared_gate_sb")]


class LayerConfig(C.Structure):
    _fields_ = [(n, INT) for n in ("hidden", "experts", "top_k", "expert_width", "group_size", "heads",
                                   "kv_heads", "head_dim", "rot_dims", "index_dim")] + [
        ("rope_theta", F32), ("eps", F32), ("max_positions", I64)]


class LayerWeights(C.Structure):
    _fields_ = [(n, P) for n in ("attn_norm", "post_norm", "qkv_w", "qkv_s", "qkv_b", "q_norm", "k_norm",
                                 "o_w", "o_s", "o_b", "rope_cos", "rope_sin")] + [
        ("moe", MoEWeights), ("qkv_rows", INT), ("qkv_sb", P), ("o_sb", P)]


class Q4(C.Structure):
    _fields_ = [("w", P), ("s", P), ("b", P), ("sb", P)]


class HCWeights(C.Structure):
    _fields_ = [("norm_scale", P), ("down", Q4), ("inject", Q4), ("up", Q4)]


class HeadConfig(C.Structure):
    _fields_ = [("layer", LayerConfig), ("hc", INT), ("lowrank", INT), ("vocab", I64), ("shortlist_low", INT),
                ("shortlist_special_from", I64)]


class HeadWeights(C.Structure):
    _fields_ = [("embed", Q4), ("pre_norm_embedding", P), ("pre_norm_hidden", P), ("fc_embedding", Q4),
                ("fc_hidden", Q4), ("attn_hc", HCWeights), ("mlp_hc", HCWeights), ("final_hc", HCWeights),
                ("layer", LayerWeights), ("shortlist", Q4), ("shortlist_ids", P), ("shortlist_rows", INT)]


class ForceParams(C.Structure):
    _fields_ = [("teacher", P), ("teacher_len", I64), ("rate", F32), ("seed", U64)]


class DrafterInfo(C.Structure):
    _fields_ = [(n, I64) for n in ("cache_offset", "committed_inputs", "staged_inputs", "backlog_inputs",
                                   "round_base_offset", "round_valid_offset")] + [
        (n, INT) for n in ("round_in_flight", "round_draft_steps", "has_frontier", "released")]


class GDNConfig(C.Structure):
    _fields_ = [("hidden", INT), ("key_heads", INT), ("value_heads", INT), ("conv_kernel", INT),
                ("group_size", INT), ("eps", C.c_float)]


class GDNWeights(C.Structure):
    _fields_ = [("in_proj", Q4), ("conv_w", P), ("neg_exp_alog", P), ("dt_bias", P), ("norm_w", P),
                ("out_proj", Q4)]


PLE_MAX_NGRAM = 8
PLE_MAX_HEADS = 32


class PLEConfig(C.Structure):
    _fields_ = [("hidden", INT), ("hc", INT), ("embed_dim", INT), ("ngram_size", INT), ("heads_per_ngram", INT),
                ("conv_kernel", INT), ("group_size", INT), ("row_group_size", INT), ("eos", I32),
                ("vocab_base", I64), ("token_vocab", I64), ("eps", C.c_float)]


class NGramTable(C.Structure):
    _fields_ = [("w", P), ("s", P), ("b", P), ("rows", I64), ("multiplier", I64 * PLE_MAX_NGRAM),
                ("vocab", I64 * PLE_MAX_HEADS), ("offset", I64 * PLE_MAX_HEADS)]


class PLEWeights(C.Structure):
    _fields_ = [("key_proj", Q4), ("value_proj", Q4), ("norm_key", P), ("norm_query", P), ("norm_conv", P),
                ("conv_w", P), ("table", NGramTable)]


class TargetConfig(C.Structure):
    _fields_ = [("layer", LayerConfig), ("key_heads", INT), ("value_heads", INT), ("conv_kernel", INT),
                ("num_layers", INT), ("full_attention_interval", INT), ("hc", INT), ("lowrank", INT),
                ("vocab", I64), ("ple_layer", INT), ("ple", PLEConfig)]


class TargetLayerWeights(C.Structure):
    _fields_ = [("kind", INT), ("attn", LayerWeights), ("gdn", GDNWeights), ("attn_hc", HCWeights),
                ("mlp_hc", HCWeights), ("ple", PLEWeights)]


class TargetWeights(C.Structure):
    _fields_ = [("embed", Q4), ("final_hc", HCWeights), ("lm_head", Q4)]


_SIGS = {
    "mtpx_last_error": (C.c_char_p, []),
    "mtpx_version": (C.c_char_p, []),
    "mtpx_ctx_new": (INT, [C.POINTER(Handle), INT]),
    "mtpx_ctx_free": (INT, [Handle]),
    "mtpx_ctx_set_stream": (INT, [Handle, P]),
    "mtpx_ctx_use_own_stream": (INT, [Handle]),
    "mtpx_ctx_synchronize": (INT, [Handle]),
    "mtpx_affine_quantize": (INT, [Handle, P, I64, INT, INT, P, P, P]),
    "mtpx_randn_bf16": (INT, [Handle, P, I64, U64, U32, F32]),
    "mtpx_q4_sb_row_len": (INT, [INT, INT]),
    "mtpx_q4_pack_sb": (INT, [Handle, P, P, I64, INT, INT, P]),
    "mtpx_qmv": (INT, [Handle, P, P, P, P, INT, INT, INT, P, INT, P, P]),
    "mtpx_moe_forward": (INT, [Handle, C.POINTER(MoEWeights), P, INT, P, P, P, P, P]),
    "mtpx_moe_forward_noalloc": (INT, [Handle, C.POINTER(MoEWeights), P, INT, P, P, P, P, P]),
    "mtpx_attn_prep": (INT, [Handle, P, INT, INT, INT, INT, INT, INT, P, P, F32, P, P, INT, P, P, P, I64]),
    "mtpx_attn_verify": (INT, [Handle, P, INT, INT, INT, INT, P, P, I64, INT, F32, P, INT, INT, P, P]),
    "mtpx_rmsnorm": (INT, [Handle, P, P, INT, INT, P, F32, P, P]),
    "mtpx_kv_new": (INT, [Handle, INT, INT, I64, C.POINTER(Handle)]),
    "mtpx_kv_free": (INT, [Handle]),
    "mtpx_kv_offset": (INT, [Handle, C.POINTER(I64)]),
    "mtpx_kv_set_offset": (INT, [Handle, I64]),
    "mtpx_kv_trim": (INT, [Handle, I64, C.POINTER(I64)]),
    "mtpx_kv_buffers": (INT, [Handle, C.POINTER(P), C.POINTER(P), C.POINTER(I64)]),
    "mtpx_argmax_rows": (INT, [Handle, P, INT, I64, P]),
    "mtpx_accept_greedy": (INT, [Handle, P, INT, I64, P, I32, P]),
    "mtpx_accept_sample": (INT, [Handle, P, P, INT, I64, P, F32, U64, U64, I32, P]),
    "mtpx_accept_sample_bf16": (INT, [Handle, P, P, INT, I64, P, F32, U64, U64, I32, P, P]),
    "mtpx_top_two": (INT, [Handle, P, INT, I64, P, P]),
    "mtpx_st_open": (INT, [C.c_char_p, C.POINTER(Handle)]),
    "mtpx_st_free": (INT, [Handle]),
    "mtpx_st_count": (INT, [Handle, C.POINTER(I64)]),
    "mtpx_st_tensor": (INT, [Handle, I64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(INT),
                             C.POINTER(C.POINTER(I64)), C.POINTER(I64)]),
    "mtpx_st_find": (INT, [Handle, C.c_char_p, C.POINTER(I64)]),
    "mtpx_st_metadata": (INT, [Handle, C.c_char_p, C.POINTER(C.c_char_p)]),
    "mtpx_st_read": (INT, [Handle, I64, P, I64]),
    "mtpx_checkpoint_open": (INT, [C.POINTER(C.c_char_p), INT, C.POINTER(Handle)]),
    "mtpx_checkpoint_free": (INT, [Handle]),
    "mtpx_checkpoint_count": (INT, [Handle, C.POINTER(I64)]),
    "mtpx_target_load": (INT, [Handle, C.POINTER(TargetConfig), Handle, C.c_char_p, INT, C.POINTER(Handle)]),
    "mtpx_head_load": (INT, [Handle, C.POINTER(HeadConfig), Handle, Handle, C.c_char_p, INT, C.POINTER(Handle)]),
    "mtpx_top_two_bf16": (INT, [Handle, P, INT, I64, P, P]),
    "mtpx_accept_greedy_bf16": (INT, [Handle, P, INT, I64, P, I32, P, P, P]),
    "mtpx_force_draft": (INT, [Handle, P, P, I64, F32, U64]),
    "mtpx_session_new": (INT, [Handle, Handle, Handle, C.POINTER(Handle)]),
    "mtpx_session_free": (INT, [Handle]),
    "mtpx_session_reset": (INT, [Handle]),
    "mtpx_session_prefill": (INT, [Handle, P, INT, C.POINTER(I32)]),
    "mtpx_round": (INT, [Handle, INT, C.POINTER(ForceParams), P, C.POINTER(INT)]),
    "mtpx_round_sampled": (INT, [Handle, INT, C.POINTER(ForceParams), F32, U64, P, C.POINTER(INT)]),
    "mtpx_session_info": (INT, [Handle, C.POINTER(I64), C.POINTER(Handle), C.POINTER(Handle)]),
    "mtpx_layer_new_random": (INT, [Handle, C.POINTER(LayerConfig), U64, C.POINTER(Handle)]),
    "mtpx_layer_free": (INT, [Handle]),
    "mtpx_layer_weights_get": (INT, [Handle, C.POINTER(LayerWeights)]),
    "mtpx_layer_forward": (INT, [Handle, Handle, Handle, P, INT, P]),
    "mtpx_last_moe_bytes": (INT, [Handle, C.POINTER(I64), C.POINTER(I32)]),
    "mtpx_shortlist_argmax": (INT, [Handle, P, INT, P, P, P, P, INT, INT, P, P]),
    "mtpx_head_new_random": (INT, [Handle, C.POINTER(HeadConfig), U64, C.POINTER(Handle)]),
    "mtpx_head_free": (INT, [Handle]),
    "mtpx_head_weights_get": (INT, [Handle, C.POINTER(HeadWeights)]),
    "mtpx_head_forward": (INT, [Handle, Handle, Handle, P, INT, P, P, P, P]),
    "mtpx_drafter_new": (INT, [Handle, Handle, C.POINTER(Handle)]),
    "mtpx_drafter_free": (INT, [Handle]),
    "mtpx_drafter_observe": (INT, [Handle, P, P, INT]),
    "mtpx_drafter_step": (INT, [Handle, P, P, P, P]),
    "mtpx_drafter_finalize": (INT, [Handle, INT, P, P, INT]),
    "mtpx_drafter_discard": (INT, [Handle]),
    "mtpx_drafter_release": (INT, [Handle]),
    "mtpx_drafter_info_get": (INT, [Handle, C.POINTER(DrafterInfo)]),
    "mtpx_drafter_bytes_per_token": (INT, [Handle, C.POINTER(I64)]),
    "mtpx_gdn_new_random": (INT, [Handle, C.POINTER(GDNConfig), U64, C.POINTER(Handle)]),
    "mtpx_gdn_free": (INT, [Handle]),
    "mtpx_gdn_weights_get": (INT, [Handle, C.POINTER(GDNWeights)]),
    "mtpx_gdn_state_new": (INT, [Handle, C.POINTER(GDNConfig), C.POINTER(Handle)]),
    "mtpx_gdn_state_free": (INT, [Handle]),
    "mtpx_gdn_state_load": (INT, [Handle, Handle, P, P]),
    "mtpx_gdn_state_store": (INT, [Handle, Handle, P, P]),
    "mtpx_gdn_commit": (INT, [Handle, INT]),
    "mtpx_gdn_state_info": (INT, [Handle, C.POINTER(INT), C.POINTER(INT)]),
    "mtpx_gdn_core": (INT, [Handle, Handle, Handle, P, INT, P]),
    "mtpx_gdn_forward": (INT, [Handle, Handle, Handle, P, INT, P, P]),
    "mtpx_ple_new_random": (INT, [Handle, C.POINTER(PLEConfig), U64, C.POINTER(Handle)]),
    "mtpx_ple_free": (INT, [Handle]),
    "mtpx_ple_weights_get": (INT, [Handle, C.POINTER(PLEWeights)]),
    "mtpx_ple_state_new": (INT, [Handle, C.POINTER(PLEConfig), C.POINTER(Handle)]),
    "mtpx_ple_state_free": (INT, [Handle]),
    "mtpx_ple_state_load": (INT, [Handle, Handle, P, P]),
    "mtpx_ple_state_store": (INT, [Handle, Handle, P, P]),
    "mtpx_ple_commit": (INT, [Handle, INT]),
    "mtpx_ple_state_info": (INT, [Handle, C.POINTER(INT), C.POINTER(INT)]),
    "mtpx_ngram_row_ids": (INT, [Handle, Handle, P, INT, P]),
    "mtpx_ple_forward": (INT, [Handle, Handle, Handle, P, INT, P, P, P, P]),
    "mtpx_target_state_ple": (INT, [Handle, C.POINTER(Handle)]),
    "mtpx_target_new_random": (INT, [Handle, C.POINTER(TargetConfig), U64, C.POINTER(Handle)]),
    "mtpx_target_free": (INT, [Handle]),
    "mtpx_target_adopt": (INT, [Handle, C.POINTER(TargetConfig), C.POINTER(TargetWeights),
                                C.POINTER(TargetLayerWeights), INT, C.POINTER(Handle)]),
    "mtpx_head_adopt": (INT, [Handle, C.POINTER(HeadConfig), C.POINTER(HeadWeights), INT, C.POINTER(Handle)]),
    "mtpx_target_weights_get": (INT, [Handle, C.POINTER(TargetWeights)]),
    "mtpx_target_layer_weights_get": (INT, [Handle, INT, C.POINTER(TargetLayerWeights)]),
    "mtpx_target_state_new": (INT, [Handle, Handle, C.POINTER(Handle)]),
    "mtpx_target_state_free": (INT, [Handle]),
    "mtpx_target_state_kv": (INT, [Handle, INT, C.POINTER(Handle)]),
    "mtpx_target_state_gdn": (INT, [Handle, INT, C.POINTER(Handle)]),
    "mtpx_target_state_set_offset": (INT, [Handle, I64]),
    "mtpx_target_state_info": (INT, [Handle, C.POINTER(I64), C.POINTER(INT)]),
    "mtpx_target_state_reset": (INT, [Handle, Handle]),
    "mtpx_target_verify": (INT, [Handle, Handle, Handle, P, INT, P, P, P]),
    "mtpx_target_commit": (INT, [Handle, INT]),
    "mtpx_target_prefill": (INT, [Handle, Handle, Handle, P, INT, P, P]),
    "mtpx_target_moe_unique": (INT, [Handle, Handle, P]),
    "mtpx_profile_enable": (INT, [Handle, INT]),
    "mtpx_profile_reset": (INT, [Handle]),
    "mtpx_profile_dump": (INT, [Handle, C.c_char_p, C.c_size_t]),
}

_LIB = None


class MtpxError(RuntimeError):
    pass


def header_symbols() -> list[str]:
    """Every entry point declared in include/mtpx.h."""
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(mtpx_\w+)\s*\(", txt, re.M)))


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise MtpxError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = lib().mtpx_last_error().decode(errors="replace")
        raise MtpxError(f"{what} failed (code {rc}): {msg}")
