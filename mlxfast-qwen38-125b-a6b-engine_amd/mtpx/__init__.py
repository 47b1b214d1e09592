"""mtpx -- Python host binding of the MI355X MTP speculative-decode step.

Thin wrappers over the C ABI (include/mtpx.h).  torch is used only to own
device memory: every compute call goes to libmtpx.so's HIP kernels; if the
library is missing the import of any op raises.

bf16 tensors are torch.bfloat16 (the C ABI sees their uint16 bit patterns).
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import (DrafterInfo, ForceParams, GDNConfig, GDNWeights, Handle, HCWeights, HeadConfig, HeadWeights, LayerConfig,
                   LayerWeights, MoEWeights, MtpxError, NGramTable, PLEConfig, PLEWeights, Q4, TargetConfig,
                   TargetLayerWeights, TargetWeights, check)

__all__ = ["Context", "KVCache", "DecoderLayer", "MTPHead", "Drafter", "GDN", "GDNState", "PLE", "PLEState", "Target",
           "TargetState", "Session", "SafetensorsFile", "Checkpoint", "MoEWeights", "LayerConfig", "HeadConfig", "GDNConfig", "PLEConfig", "TargetConfig",
           "MtpxError", "moe_weights_from"]


def _ptr(t):
    """A tensor's device address (or a raw address given as int)."""
    if t is None:
        return None
    if isinstance(t, int):
        return C.c_void_p(t)
    assert t.is_contiguous(), "row-contiguous tensors only"
    return C.c_void_p(t.data_ptr())


class Context:
    """A device, a HIP stream and a reusable workspace (mtpx_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.lib()
        self.h = Handle()
        check(self.lib.mtpx_ctx_new(C.byref(self.h), device), "mtpx_ctx_new")
        self.device = device
        # run on torch's current stream so torch's fills and copies are ordered with the kernels
        import torch
        self.set_stream(torch.cuda.current_stream(device).cuda_stream)

    def set_stream(self, stream: int):
        check(self.lib.mtpx_ctx_set_stream(self.h, C.c_void_p(stream) if stream else None), "set_stream")

    def close(self):
        if self.h.ctx:
            self.lib.mtpx_ctx_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        check(self.lib.mtpx_ctx_synchronize(self.h), "synchronize")

    # -- kernels ---------------------------------------------------------------------------
    def affine_quantize(self, w, gs, wq, s, b):
        K = w.shape[-1]
        check(self.lib.mtpx_affine_quantize(self.h, _ptr(w), w.numel() // K, K, gs, _ptr(wq), _ptr(s), _ptr(b)),
              "affine_quantize")

    def randn_bf16(self, out, seed, tensor, sigma):
        check(self.lib.mtpx_randn_bf16(self.h, _ptr(out), out.numel(), seed, tensor, sigma), "randn_bf16")

    def qmv(self, wq, s, b, gs, x, y, yf=None, sb=None):
        K = x.shape[-1]
        M = x.numel() // K
        N = wq.numel() // (K // 8)
        check(self.lib.mtpx_qmv(self.h, _ptr(wq), _ptr(s), _ptr(b), _ptr(sb), N, K, gs, _ptr(x), M, _ptr(y),
                                _ptr(yf)), "qmv")

    def sb_row_len(self, K: int, gs: int) -> int:
        n = self.lib.mtpx_q4_sb_row_len(K, gs)
        if n < 0:
            check(1, "q4_sb_row_len")
        return n

    def pack_sb(self, s, b, K: int, gs: int, out=None):
        """Packed (scale, bias) rows of a q4 matrix (int32 tensor [rows, sb_row_len])."""
        import torch
        rows = s.numel() // (K // gs)
        if out is None:
            out = torch.empty(rows, self.sb_row_len(K, gs), dtype=torch.int32, device=s.device)
        check(self.lib.mtpx_q4_pack_sb(self.h, _ptr(s), _ptr(b), rows, K, gs, _ptr(out)), "q4_pack_sb")
        return out

    def moe_forward(self, w: MoEWeights, x, y, idx=None, wts=None, logits=None, n_unique=None):
        M = x.shape[0]
        check(self.lib.mtpx_moe_forward(self.h, C.byref(w), _ptr(x), M, _ptr(y), _ptr(idx), _ptr(wts),
                                        _ptr(logits), _ptr(n_unique)), "moe_forward")

    def moe_forward_noalloc(self, w: MoEWeights, x, y, idx=None, wts=None, logits=None, n_unique=None):
        M = x.shape[0]
        check(self.lib.mtpx_moe_forward_noalloc(self.h, C.byref(w), _ptr(x), M, _ptr(y), _ptr(idx), _ptr(wts),
                                                _ptr(logits), _ptr(n_unique)), "moe_forward_noalloc")

    def attn_prep(self, qkv, HQ, HK, D, rot, qnorm, knorm, eps, cos_t, sin_t, pos0, q, kcache, vcache,
                  tmax=None):
        S, QW = qkv.shape
        tmax = kcache.shape[1] if tmax is None else tmax
        check(self.lib.mtpx_attn_prep(self.h, _ptr(qkv), S, QW, HQ, HK, D, rot, _ptr(qnorm), _ptr(knorm), eps,
                                      _ptr(cos_t), _ptr(sin_t), pos0, _ptr(q), _ptr(kcache), _ptr(vcache), tmax),
              "attn_prep")

    def attn_verify(self, q, kcache, vcache, T, scale, out=None, qkv=None, gate_off=0, out_gated=None,
                    HK=None, tmax=None):
        S, HQ, D = q.shape
        if HK is None:
            HK, tmax, _ = kcache.shape
        QW = qkv.shape[1] if qkv is not None else 0
        check(self.lib.mtpx_attn_verify(self.h, _ptr(q), S, HQ, HK, D, _ptr(kcache), _ptr(vcache), tmax, T,
                                        scale, _ptr(qkv), QW, gate_off, _ptr(out), _ptr(out_gated)),
              "attn_verify")

    def rmsnorm(self, x, w, eps, y, resid=None, sum_out=None):
        M, H = x.shape
        check(self.lib.mtpx_rmsnorm(self.h, _ptr(x), _ptr(resid), M, H, _ptr(w), eps, _ptr(sum_out), _ptr(y)),
              "rmsnorm")

    def argmax_rows(self, x, out):
        rows, V = x.shape
        check(self.lib.mtpx_argmax_rows(self.h, _ptr(x), rows, V, _ptr(out)), "argmax_rows")

    def top_two(self, logits, ids, values):
        """ids int32 [rows, 2], values f32 [rows, 2]: each row's two best entries (argmax order)."""
        rows, V = logits.shape
        fn = self.lib.mtpx_top_two_bf16 if logits.dtype.itemsize == 2 else self.lib.mtpx_top_two
        check(fn(self.h, _ptr(logits), rows, V, _ptr(ids), _ptr(values)), "top_two")

    def accept_greedy(self, logits, drafts, kv_offset, out3):
        k = drafts.numel()
        check(self.lib.mtpx_accept_greedy(self.h, _ptr(logits), k, logits.shape[1], _ptr(drafts), kv_offset,
                                          _ptr(out3)), "accept_greedy")

    def accept_greedy_bf16(self, logits, drafts, kv_offset, out3, argmax_out=None, tokens_out=None):
        k = 0 if drafts is None else drafts.numel()
        check(self.lib.mtpx_accept_greedy_bf16(self.h, _ptr(logits), k, logits.shape[1], _ptr(drafts), kv_offset,
                                               _ptr(out3), _ptr(argmax_out), _ptr(tokens_out)), "accept_greedy_bf16")

    def force_draft(self, token, teacher, pos, p, seed):
        check(self.lib.mtpx_force_draft(self.h, _ptr(token), _ptr(teacher), pos, p, seed), "force_draft")

    def accept_sample(self, tlogits, dlogits, drafts, temperature, seed, offset, kv_offset, out3):
        """dlogits None: one-hot draft distributions at the drafts (a greedy drafter)."""
        k = drafts.numel()
        check(self.lib.mtpx_accept_sample(self.h, _ptr(tlogits), _ptr(dlogits), k, tlogits.shape[1],
                                          _ptr(drafts), temperature, seed, offset, kv_offset, _ptr(out3)),
              "accept_sample")

    def accept_sample_bf16(self, tlogits, dlogits, drafts, temperature, seed, offset, kv_offset, out3,
                           tokens_out=None):
        k = drafts.numel()
        check(self.lib.mtpx_accept_sample_bf16(self.h, _ptr(tlogits), _ptr(dlogits), k, tlogits.shape[1],
                                               _ptr(drafts), temperature, seed, offset, kv_offset, _ptr(out3),
                                               _ptr(tokens_out)), "accept_sample_bf16")

    def shortlist_argmax(self, x, w, s, b, gs, ids, out, sb=None):
        """out[0] = ids[argmax_j bf16(W_j . x)] over the shortlist rows (lowest position on ties)."""
        check(self.lib.mtpx_shortlist_argmax(self.h, _ptr(x), x.shape[-1], _ptr(w), _ptr(s), _ptr(b), _ptr(sb), gs,
                                             ids.shape[0], _ptr(ids), _ptr(out)), "shortlist_argmax")

    def profile(self, on: bool = True):
        check(self.lib.mtpx_profile_enable(self.h, 1 if on else 0), "profile_enable")

    def profile_reset(self):
        check(self.lib.mtpx_profile_reset(self.h), "profile_reset")

    def profile_stats(self) -> dict:
        """{kernel: (launches, total_ms)} from the events recorded on the context stream."""
        buf = C.create_string_buffer(1 << 16)
        check(self.lib.mtpx_profile_dump(self.h, buf, len(buf)), "profile_dump")
        out = {}
        for line in buf.value.decode().splitlines():
            name, n, ms = line.split()
            out[name] = (int(n), float(ms))
        return out

    def last_moe_bytes(self):
        b = C.c_int64()
        nu = C.c_int32()
        check(self.lib.mtpx_last_moe_bytes(self.h, C.byref(b), C.byref(nu)), "last_moe_bytes")
        return b.value, nu.value


class KVCache:
    """Contiguous bf16 K/V [kv_heads, tmax, head_dim] with offset rollback (mtpx_kv)."""

    def __init__(self, ctx: Context, kv_heads: int, head_dim: int, tmax: int):
        self.ctx = ctx
        self.h = Handle()
        check(ctx.lib.mtpx_kv_new(ctx.h, kv_heads, head_dim, tmax, C.byref(self.h)), "kv_new")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_kv_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def offset(self) -> int:
        o = C.c_int64()
        check(self.ctx.lib.mtpx_kv_offset(self.h, C.byref(o)), "kv_offset")
        return o.value

    @offset.setter
    def offset(self, v: int):
        check(self.ctx.lib.mtpx_kv_set_offset(self.h, v), "kv_set_offset")

    def trim(self, n: int) -> int:
        t = C.c_int64()
        check(self.ctx.lib.mtpx_kv_trim(self.h, n, C.byref(t)), "kv_trim")
        return t.value

    def buffers(self):
        k, v, tmax = C.c_void_p(), C.c_void_p(), C.c_int64()
        check(self.ctx.lib.mtpx_kv_buffers(self.h, C.byref(k), C.byref(v), C.byref(tmax)), "kv_buffers")
        return k.value, v.value, tmax.value


class DecoderLayer:
    """One full-shape attention + MoE decoder layer with seeded random weights (mtpx_layer)."""

    def __init__(self, ctx: Context, cfg: LayerConfig, seed: int):
        self.ctx = ctx
        self.cfg = cfg
        self.h = Handle()
        check(ctx.lib.mtpx_layer_new_random(ctx.h, C.byref(cfg), seed, C.byref(self.h)), "layer_new_random")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_layer_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weights(self) -> LayerWeights:
        w = LayerWeights()
        check(self.ctx.lib.mtpx_layer_weights_get(self.h, C.byref(w)), "layer_weights_get")
        return w

    def forward(self, kv: KVCache, x, y):
        check(self.ctx.lib.mtpx_layer_forward(self.ctx.h, self.h, kv.h, _ptr(x), x.shape[0], _ptr(y)),
              "layer_forward")


class MTPHead:
    """The MTP head (embedding, two projections, one attention + MoE layer between
    hyper-connection mixers, shortlist lm_head) with seeded random weights (mtpx_head)."""

    def __init__(self, ctx: Context, cfg: HeadConfig, seed: int):
        self.ctx = ctx
        self.cfg = cfg
        self.h = Handle()
        check(ctx.lib.mtpx_head_new_random(ctx.h, C.byref(cfg), seed, C.byref(self.h)), "head_new_random")

    @classmethod
    def adopt(cls, ctx: Context, cfg: HeadConfig, weights: HeadWeights, pack_sb: bool = True):
        """A head over caller-owned device weights (mtpx_head_adopt; the tensors must outlive it)."""
        hd = cls.__new__(cls)
        hd.ctx, hd.cfg, hd.h = ctx, cfg, Handle()
        check(ctx.lib.mtpx_head_adopt(ctx.h, C.byref(cfg), C.byref(weights), 1 if pack_sb else 0, C.byref(hd.h)),
              "head_adopt")
        return hd

    @classmethod
    def load(cls, ctx: Context, cfg: HeadConfig, ckpt: "Checkpoint", target: "Target", prefix: "str | None" = None,
             pack_sb: bool = True):
        """The checkpoint's MTP head over `target` (mtpx_head_load; the target must outlive it)."""
        hd = cls.__new__(cls)
        hd.ctx, hd.cfg, hd.h = ctx, cfg, Handle()
        check(ctx.lib.mtpx_head_load(ctx.h, C.byref(cfg), ckpt.h, target.h,
                                     prefix.encode() if prefix is not None else None, 1 if pack_sb else 0,
                                     C.byref(hd.h)), "head_load")
        return hd

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_head_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weights(self) -> HeadWeights:
        w = HeadWeights()
        check(self.ctx.lib.mtpx_head_weights_get(self.h, C.byref(w)), "head_weights_get")
        return w

    def forward(self, kv: KVCache, ids, multi, multi_next, sample=None, draft=None):
        """One draft step over S = len(ids) inputs; advances the head cache by S."""
        check(self.ctx.lib.mtpx_head_forward(self.ctx.h, self.h, kv.h, _ptr(ids), ids.shape[0], _ptr(multi),
                                             _ptr(multi_next), _ptr(sample), _ptr(draft)), "head_forward")


class Drafter:
    """Per-request MTP drafter state (mtpx_drafter): the head's own KV cache plus the
    trusted target transitions not yet in it; the CBv2 request-stateful drafter
    protocol (observe / step / finalize / discard / release)."""

    MAX_DEPTH = 6

    def __init__(self, ctx: Context, head: MTPHead):
        self.ctx = ctx
        self.head = head
        self.h = Handle()
        check(ctx.lib.mtpx_drafter_new(ctx.h, head.h, C.byref(self.h)), "drafter_new")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_drafter_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def observe(self, tokens, multi):
        check(self.ctx.lib.mtpx_drafter_observe(self.h, _ptr(tokens), _ptr(multi), tokens.shape[0]), "drafter_observe")

    def step(self, token, multi, draft, multi_out):
        check(self.ctx.lib.mtpx_drafter_step(self.h, _ptr(token), _ptr(multi), _ptr(draft), _ptr(multi_out)),
              "drafter_step")

    def finalize(self, confirmed_inputs: int, tokens=None, multi=None):
        n = 0 if tokens is None else tokens.shape[0]
        check(self.ctx.lib.mtpx_drafter_finalize(self.h, confirmed_inputs, _ptr(tokens), _ptr(multi), n),
              "drafter_finalize")

    def discard(self):
        check(self.ctx.lib.mtpx_drafter_discard(self.h), "drafter_discard")

    def release(self):
        check(self.ctx.lib.mtpx_drafter_release(self.h), "drafter_release")

    def info(self) -> dict:
        i = DrafterInfo()
        check(self.ctx.lib.mtpx_drafter_info_get(self.h, C.byref(i)), "drafter_info")
        return {n: getattr(i, n) for n, _ in DrafterInfo._fields_}

    def bytes_per_token(self) -> int:
        v = C.c_int64()
        check(self.ctx.lib.mtpx_drafter_bytes_per_token(self.head.h, C.byref(v)), "drafter_bytes_per_token")
        return v.value


class GDN:
    """A gated-deltanet sublayer with seeded random weights (mtpx_gdn)."""

    def __init__(self, ctx: Context, cfg: GDNConfig, seed: int):
        self.ctx = ctx
        self.cfg = cfg
        self.h = Handle()
        check(ctx.lib.mtpx_gdn_new_random(ctx.h, C.byref(cfg), seed, C.byref(self.h)), "gdn_new_random")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_gdn_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weights(self) -> GDNWeights:
        w = GDNWeights()
        check(self.ctx.lib.mtpx_gdn_weights_get(self.h, C.byref(w)), "gdn_weights_get")
        return w

    def core(self, state: "GDNState", proj, gated):
        check(self.ctx.lib.mtpx_gdn_core(self.ctx.h, self.h, state.h, _ptr(proj), proj.shape[0], _ptr(gated)),
              "gdn_core")

    def forward(self, state: "GDNState", x, y, gated=None):
        check(self.ctx.lib.mtpx_gdn_forward(self.ctx.h, self.h, state.h, _ptr(x), x.shape[0], _ptr(y), _ptr(gated)),
              "gdn_forward")


class GDNState:
    """Committed conv rows + recurrent state of one GDN layer for one request, with the
    journal of the last window (mtpx_gdn_state)."""

    def __init__(self, ctx: Context, cfg: GDNConfig):
        self.ctx = ctx
        self.h = Handle()
        check(ctx.lib.mtpx_gdn_state_new(ctx.h, C.byref(cfg), C.byref(self.h)), "gdn_state_new")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_gdn_state_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load(self, conv, ssm):
        check(self.ctx.lib.mtpx_gdn_state_load(self.ctx.h, self.h, _ptr(conv), _ptr(ssm)), "gdn_state_load")

    def store(self, conv, ssm):
        check(self.ctx.lib.mtpx_gdn_state_store(self.ctx.h, self.h, _ptr(conv), _ptr(ssm)), "gdn_state_store")

    def commit(self, n: int):
        check(self.ctx.lib.mtpx_gdn_commit(self.h, n), "gdn_commit")

    def info(self):
        w, c = C.c_int(), C.c_int()
        check(self.ctx.lib.mtpx_gdn_state_info(self.h, C.byref(w), C.byref(c)), "gdn_state_info")
        return w.value, c.value


class PLE:
    """The PLE n-gram block with seeded random weights and a resident row table (mtpx_ple)."""

    def __init__(self, ctx: Context, cfg: PLEConfig, seed: int):
        self.ctx = ctx
        self.cfg = cfg
        self.h = Handle()
        check(ctx.lib.mtpx_ple_new_random(ctx.h, C.byref(cfg), seed, C.byref(self.h)), "ple_new_random")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_ple_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weights(self) -> PLEWeights:
        w = PLEWeights()
        check(self.ctx.lib.mtpx_ple_weights_get(self.h, C.byref(w)), "ple_weights_get")
        return w

    def row_ids(self, history, S: int, out):
        check(self.ctx.lib.mtpx_ngram_row_ids(self.ctx.h, self.h, _ptr(history), S, _ptr(out)), "ngram_row_ids")

    def forward(self, state: "PLEState", ids, stream, out=None, sum=None, embedded=None):
        check(self.ctx.lib.mtpx_ple_forward(self.ctx.h, self.h, state.h, _ptr(ids), ids.shape[0], _ptr(stream),
                                            _ptr(out), _ptr(sum), _ptr(embedded)), "ple_forward")


class PLEState:
    """Carried conv rows + token context of the PLE block for one request, with the last
    window (mtpx_ple_state)."""

    def __init__(self, ctx: Context, cfg: PLEConfig):
        self.ctx = ctx
        self.h = Handle()
        check(ctx.lib.mtpx_ple_state_new(ctx.h, C.byref(cfg), C.byref(self.h)), "ple_state_new")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_ple_state_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load(self, conv, context):
        check(self.ctx.lib.mtpx_ple_state_load(self.ctx.h, self.h, _ptr(conv), _ptr(context)), "ple_state_load")

    def store(self, conv, context):
        check(self.ctx.lib.mtpx_ple_state_store(self.ctx.h, self.h, _ptr(conv), _ptr(context)), "ple_state_store")

    def commit(self, n: int):
        check(self.ctx.lib.mtpx_ple_commit(self.h, n), "ple_commit")

    def info(self):
        w, c = C.c_int(), C.c_int()
        check(self.ctx.lib.mtpx_ple_state_info(self.h, C.byref(w), C.byref(c)), "ple_state_info")
        return w.value, c.value


def _borrowed(cls, ctx, handle):
    """A wrapper around a handle owned by another object (its close() frees nothing)."""
    o = cls.__new__(cls)
    o.ctx = ctx
    o.h = Handle(handle.ctx)
    o.close = lambda: None
    return o


class Target:
    """The target model with seeded random weights (mtpx_target): embedding, the
    layer stack (GDN or attention + MoE, hyper-connection mixers), final mixer, lm_head."""

    def __init__(self, ctx: Context, cfg: TargetConfig, seed: int):
        self.ctx = ctx
        self.cfg = cfg
        self.h = Handle()
        check(ctx.lib.mtpx_target_new_random(ctx.h, C.byref(cfg), seed, C.byref(self.h)), "target_new_random")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_target_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @classmethod
    def adopt(cls, ctx: Context, cfg: TargetConfig, weights: TargetWeights, layers, pack_sb: bool = True):
        """A target over caller-owned device weights (mtpx_target_adopt; the tensors must outlive it)."""
        arr = (TargetLayerWeights * len(layers))(*layers)
        t = cls.__new__(cls)
        t.ctx, t.cfg, t.h = ctx, cfg, Handle()
        t._keep = arr
        check(ctx.lib.mtpx_target_adopt(ctx.h, C.byref(cfg), C.byref(weights), arr, 1 if pack_sb else 0,
                                        C.byref(t.h)), "target_adopt")
        return t

    @classmethod
    def load(cls, ctx: Context, cfg: TargetConfig, ckpt: "Checkpoint", prefix: "str | None" = None,
             pack_sb: bool = True):
        """A target from a safetensors checkpoint (mtpx_target_load); it owns its device copies."""
        t = cls.__new__(cls)
        t.ctx, t.cfg, t.h = ctx, cfg, Handle()
        check(ctx.lib.mtpx_target_load(ctx.h, C.byref(cfg), ckpt.h, prefix.encode() if prefix is not None else None,
                                       1 if pack_sb else 0, C.byref(t.h)), "target_load")
        return t

    def weights(self) -> TargetWeights:
        w = TargetWeights()
        check(self.ctx.lib.mtpx_target_weights_get(self.h, C.byref(w)), "target_weights_get")
        return w

    def layer_weights(self, i: int) -> TargetLayerWeights:
        w = TargetLayerWeights()
        check(self.ctx.lib.mtpx_target_layer_weights_get(self.h, i, C.byref(w)), "target_layer_weights_get")
        return w

    def verify(self, state: "TargetState", ids, logits=None, multi=None, mixed=None):
        check(self.ctx.lib.mtpx_target_verify(self.ctx.h, self.h, state.h, _ptr(ids), ids.shape[0], _ptr(logits),
                                              _ptr(multi), _ptr(mixed)), "target_verify")

    def prefill(self, state: "TargetState", ids, logits=None, multi=None):
        """S prompt tokens processed and committed; logits [vocab] of the last position, multi [S, W]."""
        check(self.ctx.lib.mtpx_target_prefill(self.ctx.h, self.h, state.h, _ptr(ids), ids.shape[0], _ptr(logits),
                                               _ptr(multi)), "target_prefill")


class TargetState:
    """Per-request caches of a Target (mtpx_target_state)."""

    def __init__(self, ctx: Context, target: Target):
        self.ctx = ctx
        self.h = Handle()
        check(ctx.lib.mtpx_target_state_new(ctx.h, target.h, C.byref(self.h)), "target_state_new")

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_target_state_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv(self, layer: int) -> KVCache:
        h = Handle()
        check(self.ctx.lib.mtpx_target_state_kv(self.h, layer, C.byref(h)), "target_state_kv")
        return _borrowed(KVCache, self.ctx, h)

    def gdn(self, layer: int) -> GDNState:
        h = Handle()
        check(self.ctx.lib.mtpx_target_state_gdn(self.h, layer, C.byref(h)), "target_state_gdn")
        return _borrowed(GDNState, self.ctx, h)

    def ple(self) -> PLEState:
        h = Handle()
        check(self.ctx.lib.mtpx_target_state_ple(self.h, C.byref(h)), "target_state_ple")
        return _borrowed(PLEState, self.ctx, h)

    def set_offset(self, offset: int):
        check(self.ctx.lib.mtpx_target_state_set_offset(self.h, offset), "target_state_set_offset")

    def info(self):
        o, w = C.c_int64(), C.c_int()
        check(self.ctx.lib.mtpx_target_state_info(self.h, C.byref(o), C.byref(w)), "target_state_info")
        return o.value, w.value

    def commit(self, n: int):
        check(self.ctx.lib.mtpx_target_commit(self.h, n), "target_commit")

    def reset(self):
        check(self.ctx.lib.mtpx_target_state_reset(self.ctx.h, self.h), "target_state_reset")

    def moe_unique(self, num_layers: int):
        out = (C.c_int32 * num_layers)()
        check(self.ctx.lib.mtpx_target_moe_unique(self.ctx.h, self.h, C.cast(out, C.c_void_p)), "target_moe_unique")
        return list(out)


def moe_weights_from(tensors: dict, H, E, K, F, gs) -> MoEWeights:
    """Build the C struct from a dict of device tensors named like its fields."""
    w = MoEWeights(H, E, K, F, gs)
    for name, _ in MoEWeights._fields_[5:]:
        t = tensors.get(name)
        setattr(w, name, t.data_ptr() if t is not None else None)
    return w


class Session:
    """One request's speculative decode (mtpx_session): prefill, then rounds of draft depth k
    (mtpx_round), each with one host readback; k = 0 is a serial decode step."""

    def __init__(self, ctx: Context, target: Target, head: "MTPHead | None" = None):
        self.ctx = ctx
        self.h = Handle()
        check(ctx.lib.mtpx_session_new(ctx.h, target.h, head.h if head is not None else Handle(), C.byref(self.h)),
              "session_new")
        self._tok = (C.c_int32 * 16)()
        self.force = None

    def close(self):
        if self.h.ctx:
            self.ctx.lib.mtpx_session_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        check(self.ctx.lib.mtpx_session_reset(self.h), "session_reset")

    def prefill(self, ids) -> int:
        first = C.c_int32()
        check(self.ctx.lib.mtpx_session_prefill(self.h, _ptr(ids), ids.shape[0], C.byref(first)), "session_prefill")
        return first.value

    def set_force(self, teacher, rate: float, seed: int):
        """Forcing hook: each draft becomes teacher[pos] with probability rate (None: off)."""
        if teacher is None:
            self.force = None
            self._teacher = None
        else:
            self._teacher = teacher
            self.force = ForceParams(teacher.data_ptr(), teacher.numel(), rate, seed)

    def round(self, k: int, temperature: float = 0.0, seed: int = 0) -> list:
        """One round; temperature > 0: speculative sampling (mtpx_round_sampled) with Philox key seed."""
        n = C.c_int()
        fp = C.byref(self.force) if self.force is not None else None
        if temperature > 0:
            check(self.ctx.lib.mtpx_round_sampled(self.h, k, fp, temperature, seed, C.cast(self._tok, C.c_void_p),
                                                  C.byref(n)), "round_sampled")
        else:
            check(self.ctx.lib.mtpx_round(self.h, k, fp, C.cast(self._tok, C.c_void_p), C.byref(n)), "round")
        return list(self._tok[:n.value])

    def offset(self) -> int:
        o = C.c_int64()
        check(self.ctx.lib.mtpx_session_info(self.h, C.byref(o), None, None), "session_info")
        return o.value

    def state(self) -> "TargetState":
        h = Handle()
        check(self.ctx.lib.mtpx_session_info(self.h, None, C.byref(h), None), "session_info")
        return _borrowed(TargetState, self.ctx, h)

    def drafter_info(self) -> dict:
        """The session drafter's counts (mtpx_drafter_info)."""
        h = Handle()
        check(self.ctx.lib.mtpx_session_info(self.h, None, None, C.byref(h)), "session_info")
        i = DrafterInfo()
        check(self.ctx.lib.mtpx_drafter_info_get(h, C.byref(i)), "drafter_info")
        return {n: getattr(i, n) for n, _ in DrafterInfo._fields_}


class SafetensorsFile:
    """One safetensors file through the library's reader (mtpx_st_*): header checked, data mapped."""

    def __init__(self, path: str):
        self.lib = _lib.lib()
        self.h = Handle()
        check(self.lib.mtpx_st_open(str(path).encode(), C.byref(self.h)), "st_open")

    def close(self):
        if self.h.ctx:
            self.lib.mtpx_st_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self) -> list:
        """[(name, dtype, shape, nbytes)] in name order."""
        n = C.c_int64()
        check(self.lib.mtpx_st_count(self.h, C.byref(n)), "st_count")
        out = []
        for i in range(n.value):
            name, dt, nd, sh, nb = C.c_char_p(), C.c_char_p(), C.c_int(), C.POINTER(C.c_int64)(), C.c_int64()
            check(self.lib.mtpx_st_tensor(self.h, i, C.byref(name), C.byref(dt), C.byref(nd), C.byref(sh),
                                          C.byref(nb)), "st_tensor")
            out.append((name.value.decode(), dt.value.decode(), tuple(sh[k] for k in range(nd.value)), nb.value))
        return out

    def read(self, name: str) -> bytes:
        i = C.c_int64()
        check(self.lib.mtpx_st_find(self.h, name.encode(), C.byref(i)), "st_find")
        nb = C.c_int64()
        check(self.lib.mtpx_st_tensor(self.h, i.value, None, None, None, None, C.byref(nb)), "st_tensor")
        buf = C.create_string_buffer(max(1, nb.value))
        check(self.lib.mtpx_st_read(self.h, i.value, buf, nb.value), "st_read")
        return buf.raw[:nb.value]

    def metadata(self, key: str):
        v = C.c_char_p()
        check(self.lib.mtpx_st_metadata(self.h, key.encode(), C.byref(v)), "st_metadata")
        return None if v.value is None else v.value.decode()


class Checkpoint:
    """Safetensors files (or directories of them) as one tensor name space (mtpx_checkpoint)."""

    def __init__(self, paths):
        if isinstance(paths, (str, bytes)):
            paths = [paths]
        self.lib = _lib.lib()
        self.h = Handle()
        arr = (C.c_char_p * len(paths))(*[str(p).encode() for p in paths])
        check(self.lib.mtpx_checkpoint_open(arr, len(paths), C.byref(self.h)), "checkpoint_open")

    def count(self) -> int:
        n = C.c_int64()
        check(self.lib.mtpx_checkpoint_count(self.h, C.byref(n)), "checkpoint_count")
        return n.value

    def close(self):
        if self.h.ctx:
            self.lib.mtpx_checkpoint_free(self.h)
            self.h.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
