"""ctypes binding of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module.  bf16 arrays are numpy ``uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = C.CDLL(path)
        _declare(_LIB)
    return _LIB


# Keys per split-KV chunk of the device's verify attention (the chunk order is
# part of its arithmetic: partials per chunk, then a fold over chunks).
ATTN_CHUNK = 32

P = C.c_void_p
I32, I64, U64, F32, F64 = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double


def _declare(L):
    sig = {
        "o_bf2f": (F32, [C.c_uint16]),
        "o_f2bf": (C.c_uint16, [F32]),
        "o_expf": (F32, [F32]),
        "o_sigmoid_bf16": (F32, [F32]),
        "o_silu_bf16": (F32, [F32]),
        "o_lanes_for_blocks": (C.c_int, [C.c_int]),
        "o_affine_quantize": (None, [P, I64, C.c_int, C.c_int, P, P, P]),
        "o_qmv": (None, [P, P, P, I64, C.c_int, C.c_int, P, C.c_int, P, P]),
        "o_xblock": (None, [P, P, P]),
        "o_router_gemv": (None, [P, C.c_int, C.c_int, P, C.c_int, P]),
        "o_topk_softmax": (None, [P, C.c_int, C.c_int, C.c_int, P, P]),
        "o_moe_block": (None, [P, P, C.c_int, P, P, P, P, P, P]),
        "o_rope_table": (None, [C.c_int, C.c_int, F64, P, P]),
        "o_attn_prep": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, P,
                               F32, P, P, C.c_int, P, P, P]),
        "o_attn_verify": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, I64, C.c_int,
                                 F32, C.c_int, P]),
        "o_attn_gate": (None, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, P]),
        "o_rmsnorm": (None, [P, C.c_int, C.c_int, P, F32, P]),
        "o_argmax_rows": (None, [P, C.c_int, I64, P]),
        "o_top2_rows": (None, [P, C.c_int, I64, P, P]),
        "o_accept_greedy": (None, [P, C.c_int, I64, P, I32, P]),
        "o_philox4x32_10": (None, [P, P, P]),
        "o_uniform": (F32, [C.c_uint32]),
        "o_accept_sample": (None, [P, P, C.c_int, I64, P, F32, U64, U64, I32, P]),
        "o_softmax_row_sum": (F32, [P, I64]),
        "o_embed_rows": (None, [P, P, P, C.c_int, C.c_int, P, C.c_int, P]),
        "o_hc_norm": (None, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, P, F32, P, P]),
        "o_silu_rows": (None, [P, I64, P]),
        "o_hc_mix": (None, [P, P, P, C.c_int, C.c_int, C.c_int, P, P]),
        "o_log1p_det": (F32, [F32]),
        "o_logaddexp0_bf16": (F32, [F32]),
        "o_sigmoid_f32": (F32, [F32]),
        "o_gdn_core": (None, [P, P, C.c_int, P, P, P, P, P, P, F32, P, P, P, P, P, P, P, P]),
        "o_ngram_row_ids": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, P, P, P, I64, I32, P]),
        "o_ple_gate": (F32, [P, P, P, P, P, P, C.c_int, F32, P, P]),
        "o_ple_conv": (None, [P, P, P, C.c_int, I64, C.c_int, C.c_int, P]),
        "o_set_threads": (None, [C.c_int]),
        "o_get_threads": (C.c_int, []),
        "o_qmm_t_bf16": (None, [P, P, P, P, C.c_int, I64, C.c_int, C.c_int, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(P)


# --------------------------------------------------------------------------- bf16 helpers
def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(h) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- wrappers
def expf(x: float) -> float:
    return lib().o_expf(x)


def lanes_for_blocks(nb: int) -> int:
    return lib().o_lanes_for_blocks(nb)


def affine_quantize(w_bf16: np.ndarray, gs: int):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = w.size // K
    wq = np.zeros(w.shape[:-1] + (K // 8,), np.uint32)
    s = np.zeros(w.shape[:-1] + (K // gs,), np.uint16)
    b = np.zeros_like(s)
    lib().o_affine_quantize(_p(w), rows, K, gs, _p(wq), _p(s), _p(b))
    return wq, s, b


def dequantize(wq, s, b, gs) -> np.ndarray:
    """float64 dequantisation s*q + b (exact); test helper."""
    wq = np.asarray(wq, np.uint32)
    K = wq.shape[-1] * 8
    q = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(wq.shape[:-1] + (K,))
    sf = np.repeat(bf16_to_f32(s).astype(np.float64), gs, axis=-1)
    bf = np.repeat(bf16_to_f32(b).astype(np.float64), gs, axis=-1)
    return sf * q + bf


def qmv(wq, s, b, gs, x_bf16):
    wq = np.ascontiguousarray(wq, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.size // (K // 8)
    y = np.zeros((M, N), np.uint16)
    yf = np.zeros((M, N), np.float32)
    lib().o_qmv(_p(wq), _p(s), _p(b), N, K, gs, _p(x), M, _p(y), _p(yf))
    return y, yf


def xblock(x32):
    x = np.ascontiguousarray(x32, np.uint16)
    m = np.zeros(32, np.int32)
    E = np.zeros(1, np.int32)
    lib().o_xblock(_p(x), _p(m), _p(E))
    return m, int(E[0])


def router_gemv(W_bf16, x_f32):
    W = np.ascontiguousarray(W_bf16, np.uint16)
    x = np.ascontiguousarray(x_f32, np.float32)
    H = W.shape[-1]
    rows = W.size // H
    M = x.size // H
    out = np.zeros((M, rows), np.float32)
    lib().o_router_gemv(_p(W), rows, H, _p(x), M, _p(out))
    return out


def topk_softmax(logits, K):
    lg = np.ascontiguousarray(logits, np.float32)
    M, E = lg.shape
    idx = np.zeros((M, K), np.int32)
    w = np.zeros((M, K), np.float32)
    lib().o_topk_softmax(_p(lg), M, E, K, _p(idx), _p(w))
    return idx, w


class MoEWeightsStruct(C.Structure):
    _fields_ = [("H", C.c_int), ("E", C.c_int), ("K", C.c_int), ("F", C.c_int), ("gs", C.c_int)] + [
        (n, P) for n in [
            "router", "shared_gate",
            "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
            "sh_gate_w", "sh_gate_s", "sh_gate_b", "sh_up_w", "sh_up_s", "sh_up_b",
            "sh_down_w", "sh_down_s", "sh_down_b", "sg_w", "sg_s", "sg_b"]]


def moe_block(w: dict, x_bf16, H, E, K, F, gs):
    """w: dict of numpy arrays named like MoEWeightsStruct fields."""
    st = MoEWeightsStruct(H, E, K, F, gs)
    keep = {}
    for name, _ in MoEWeightsStruct._fields_[5:]:
        if w.get(name) is None:  # optional: the q4 gate row (sg_*), or the bf16 row when it is given
            continue
        a = np.ascontiguousarray(w[name])
        keep[name] = a
        setattr(st, name, a.ctypes.data)
    x = np.ascontiguousarray(x_bf16, np.uint16)
    M = x.shape[0]
    y = np.zeros((M, H), np.uint16)
    idx = np.zeros((M, K), np.int32)
    wk = np.zeros((M, K), np.float32)
    logits = np.zeros((M, E), np.float32)
    gate = np.zeros(M, np.uint16)
    act = np.zeros((M * (K + 1), F), np.uint16)
    lib().o_moe_block(C.byref(st), _p(x), M, _p(y), _p(idx), _p(wk), _p(logits), _p(gate), _p(act))
    return dict(y=y, idx=idx, w=wk, logits=logits, gate=gate, act=act)


def rope_table(positions, rot, theta):
    c = np.zeros((positions, rot), np.uint16)
    s = np.zeros((positions, rot), np.uint16)
    lib().o_rope_table(positions, rot, theta, _p(c), _p(s))
    return c, s


def attn_prep(qkv, HQ, HK, D, ROT, qnorm, knorm, eps, cos_t, sin_t, pos0):
    qkv = np.ascontiguousarray(qkv, np.uint16)
    S, QW = qkv.shape
    q = np.zeros((S, HQ, D), np.uint16)
    k = np.zeros((S, HK, D), np.uint16)
    v = np.zeros((S, HK, D), np.uint16)
    lib().o_attn_prep(_p(qkv), S, QW, HQ, HK, D, ROT, _p(np.ascontiguousarray(qnorm, np.uint16)),
                      _p(np.ascontiguousarray(knorm, np.uint16)), eps,
                      _p(np.ascontiguousarray(cos_t, np.uint16)),
                      _p(np.ascontiguousarray(sin_t, np.uint16)), pos0, _p(q), _p(k), _p(v))
    return q, k, v


def attn_verify(q, kc, vc, T, scale, chunk):
    q = np.ascontiguousarray(q, np.uint16)
    S, HQ, D = q.shape
    HK, tmax, _ = kc.shape
    out = np.zeros((S, HQ, D), np.uint16)
    lib().o_attn_verify(_p(q), S, HQ, HK, D, _p(np.ascontiguousarray(kc, np.uint16)),
                        _p(np.ascontiguousarray(vc, np.uint16)), tmax, T, scale, chunk, _p(out))
    return out


def attn_gate(att, qkv, gate_off):
    att = np.ascontiguousarray(att, np.uint16)
    qkv = np.ascontiguousarray(qkv, np.uint16)
    S, width = att.shape
    out = np.zeros_like(att)
    lib().o_attn_gate(_p(att), _p(qkv), S, qkv.shape[1], gate_off, width, _p(out))
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.uint16)
    M, H = x.shape
    y = np.zeros_like(x)
    lib().o_rmsnorm(_p(x), M, H, _p(np.ascontiguousarray(w, np.uint16)), eps, _p(y))
    return y


def embed_rows(wq, s, b, gs, ids):
    """Rows ids of a q4 table, dequantized as bf16(bf16(s*q) + b)."""
    wq = np.ascontiguousarray(wq, np.uint32)
    H = wq.shape[1] * 8
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros((ids.size, H), np.uint16)
    lib().o_embed_rows(_p(wq), _p(np.ascontiguousarray(s, np.uint16)), _p(np.ascontiguousarray(b, np.uint16)),
                       H, gs, _p(ids), ids.size, _p(out))
    return out


def hc_norm(residual, out, inject, scale, hc, eps, tile=False):
    """Hyper-connection inject + group RMS norm -> (stream [S, hc*H], normed [S, hc*H])."""
    residual = np.ascontiguousarray(residual, np.uint16)
    scale = np.ascontiguousarray(scale, np.uint16)
    W = scale.size
    H = W // hc
    S = residual.shape[0]
    stream = np.zeros((S, W), np.uint16)
    normed = np.zeros((S, W), np.uint16)
    o = None if out is None else np.ascontiguousarray(out, np.uint16)
    i = None if inject is None else np.ascontiguousarray(inject, np.uint16)
    lib().o_hc_norm(_p(residual), None if o is None else _p(o), None if i is None else _p(i), S, hc, H,
                    1 if tile else 0, _p(scale), eps, _p(stream), _p(normed))
    return stream, normed


def silu_rows(x):
    x = np.ascontiguousarray(x, np.uint16)
    y = np.zeros_like(x)
    lib().o_silu_rows(_p(x), x.size, _p(y))
    return y


def hc_mix(w, normed, inj, hc):
    """Mixer combine -> (input [S, H], inject [S, hc] or None)."""
    w = np.ascontiguousarray(w, np.uint16)
    normed = np.ascontiguousarray(normed, np.uint16)
    S, W = w.shape
    H = W // hc
    inp = np.zeros((S, H), np.uint16)
    io = np.zeros((S, hc), np.uint16) if inj is not None else None
    ij = None if inj is None else np.ascontiguousarray(inj, np.uint16)
    lib().o_hc_mix(_p(w), _p(normed), None if ij is None else _p(ij), S, hc, H, _p(inp),
                   None if io is None else _p(io))
    return inp, io


def shortlist_argmax(y_bf16, ids):
    """Draft id: ids[argmax over the bf16 logits], lowest position on ties, NaN never taken
    (MLX's argmax rule, as o_argmax_rows)."""
    v = bf16_to_f32(np.asarray(y_bf16, np.uint16).reshape(1, -1))
    return int(np.asarray(ids, np.int32)[int(argmax_rows(v)[0])])


def set_threads(n: int):
    """Threads of the oracle's row-parallel loops (its results do not depend on the count)."""
    lib().o_set_threads(int(n))


def get_threads() -> int:
    return int(lib().o_get_threads())


def qmm_t_bf16(wq, scales, biases, gs, x):
    """MLX CPU _qmm_t with bf16 accumulation (the mlx_cpu timing mode) -> bf16 [M, N]."""
    wq = np.ascontiguousarray(wq, np.uint32)
    s = np.ascontiguousarray(scales, np.uint16)
    b = np.ascontiguousarray(biases, np.uint16)
    x = np.ascontiguousarray(np.atleast_2d(x), np.uint16)
    N, K = wq.shape[0], wq.shape[1] * 8
    y = np.zeros((x.shape[0], N), np.uint16)
    lib().o_qmm_t_bf16(_p(x), _p(wq), _p(s), _p(b), x.shape[0], N, K, gs, _p(y))
    return y


def argmax_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    rows, V = x.shape
    out = np.zeros(rows, np.int32)
    lib().o_argmax_rows(_p(x), rows, V, _p(out))
    return out


def top2_rows(x):
    """(ids int32 [rows, 2], values f32 [rows, 2]) in the argmax order."""
    x = np.ascontiguousarray(x, np.float32)
    rows, V = x.shape
    ids = np.zeros((rows, 2), np.int32)
    vals = np.zeros((rows, 2), np.float32)
    lib().o_top2_rows(_p(x), rows, V, _p(ids), _p(vals))
    return ids, vals


def accept_greedy(logits, drafts, kv_offset):
    lg = np.ascontiguousarray(logits, np.float32)
    d = np.ascontiguousarray(drafts, np.int32)
    k = d.size
    out = np.zeros(3, np.int32)
    lib().o_accept_greedy(_p(lg), k, lg.shape[1], _p(d), kv_offset, _p(out))
    return out


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(4, np.uint32)
    lib().o_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def uniform(r: int) -> float:
    return lib().o_uniform(r)


def accept_sample(tlogits, dlogits, drafts, temperature, seed, offset, kv_offset):
    """out3 {n, token, kv index}; dlogits None: one-hot draft distributions at the drafts."""
    t = np.ascontiguousarray(tlogits, np.float32)
    dl = None if dlogits is None else np.ascontiguousarray(dlogits, np.float32)
    d = np.ascontiguousarray(drafts, np.int32)
    out = np.zeros(3, np.int32)
    lib().o_accept_sample(_p(t), None if dl is None else _p(dl), d.size, t.shape[1], _p(d), temperature, seed,
                          offset, kv_offset, _p(out))
    return out


def softmax_row_sum(e):
    e = np.ascontiguousarray(e, np.float32)
    return lib().o_softmax_row_sum(_p(e), e.size)


# --------------------------------------------------------------------------- a20: GDN
class GDNGeom(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hk", "hv", "dk", "dv", "kc", "conv_dim", "proj_w", "z_off", "b_off",
                                         "a_off")]


def gdn_geom(hk, hv, kc=4):
    """Projection row layout qkv | z | b | a (TrackFastModel.swift:404-432)."""
    cd = (2 * hk + hv) * 128
    return GDNGeom(hk, hv, 128, 128, kc, cd, cd + hv * 128 + 2 * hv, cd, cd + hv * 128, cd + hv * 128 + hv)


def gdn_core(g, proj, conv_state, ssm, conv_w, neg_exp_alog, dt_bias, norm_w, eps=1e-6):
    """S positions of the GDN core.  Returns dict(gated, conv_state, ssm, q, k, v, y, decay, beta, delta);
    the input state arrays are not modified."""
    proj = np.ascontiguousarray(proj, np.uint16)
    S = proj.shape[0]
    cs = np.array(conv_state, np.uint16, copy=True, order="C")
    st = np.array(ssm, np.float32, copy=True, order="C")
    D = 128
    out = dict(gated=np.zeros((S, g.hv * D), np.uint16), q=np.zeros((S, g.hk * D), np.uint16),
               k=np.zeros((S, g.hk * D), np.uint16), v=np.zeros((S, g.hv * D), np.uint16),
               y=np.zeros((S, g.hv * D), np.uint16), decay=np.zeros((S, g.hv), np.float32),
               beta=np.zeros((S, g.hv), np.float32), delta=np.zeros((S, g.hv * D), np.float32))
    cw = np.ascontiguousarray(conv_w, np.uint16)
    nea = np.ascontiguousarray(neg_exp_alog, np.float32)
    dtb = np.ascontiguousarray(dt_bias, np.uint16)
    nw = np.ascontiguousarray(norm_w, np.uint16)
    lib().o_gdn_core(C.byref(g), _p(proj), S, _p(cs), _p(st), _p(cw), _p(nea), _p(dtb), _p(nw), eps,
                     _p(out["gated"]), _p(out["q"]), _p(out["k"]), _p(out["v"]), _p(out["y"]), _p(out["decay"]),
                     _p(out["beta"]), _p(out["delta"]))
    out["conv_state"] = cs
    out["ssm"] = st
    return out


# ---------------------------------------------------------------------------- PLE n-gram block
def primes_above(base: int, n: int):
    """The n consecutive primes above base (the n-gram heads' vocabulary sizes)."""
    out, v = [], base
    while len(out) < n:
        v += 1
        if v > 1 and all(v % d for d in range(2, int(v ** 0.5) + 1)):
            out.append(v)
    return out


def ngram_row_ids(history, ctx_len, ngram_size, heads_per_ngram, mult, vocab, offs, rows, eos):
    """Row ids [S, (ngram_size-1)*heads_per_ngram] of the last S = len(history) - ctx_len positions
    (-1 where an id falls outside the table)."""
    h = np.ascontiguousarray(history, np.int32)
    S = h.size - ctx_len
    nh = (ngram_size - 1) * heads_per_ngram
    out = np.zeros((S, nh), np.int32)
    lib().o_ngram_row_ids(_p(h), ctx_len, S, ngram_size, heads_per_ngram,
                          _p(np.ascontiguousarray(mult, np.int64)), _p(np.ascontiguousarray(vocab, np.int64)),
                          _p(np.ascontiguousarray(offs, np.int64)), int(rows), int(eos), _p(out))
    return out


def ple_gate(key, stream, value, kscale, qscale, cscale, eps):
    """One (position, stream) pair: -> (gated [H], normed [H], dot as float)."""
    key = np.ascontiguousarray(key, np.uint16)
    H = key.size
    gated = np.zeros(H, np.uint16)
    normed = np.zeros(H, np.uint16)
    dot = lib().o_ple_gate(_p(key), _p(np.ascontiguousarray(stream, np.uint16)),
                           _p(np.ascontiguousarray(value, np.uint16)), _p(np.ascontiguousarray(kscale, np.uint16)),
                           _p(np.ascontiguousarray(qscale, np.uint16)), _p(np.ascontiguousarray(cscale, np.uint16)),
                           H, eps, _p(gated), _p(normed))
    return gated, normed, dot


def ple_conv(full, conv_w, gated, dil):
    full = np.ascontiguousarray(full, np.uint16)
    gated = np.ascontiguousarray(gated, np.uint16)
    cw = np.ascontiguousarray(conv_w, np.uint16)
    S, W = gated.shape
    kc = cw.shape[1]
    assert full.shape == (S + (kc - 1) * dil, W)
    out = np.zeros((S, W), np.uint16)
    lib().o_ple_conv(_p(full), _p(cw), _p(gated), S, W, kc, dil, _p(out))
    return out


def ple_forward(w, cfg, stream, ids, conv_state, context):
    """The PLE block over one window (Runner/FastModel/TrackFastModel.swift:1011-1144, the three-launch
    path) on the committed state (conv_state [nb, W], context [ctx_len] int32).
    w: dict(key_proj, value_proj (q4 triples), norm_key, norm_query, norm_conv [W], conv_w [W, kc],
    table (q4 triple of [rows, row_dim]), mult, vocab, offs).
    cfg: dict(hidden, hc, ngram_size, heads_per_ngram, group_size, row_group_size, eos, eps).
    Returns dict(out, sum, row_ids, embedded, key, value, gated, normed, full, history)."""
    H, hc, n, hpn = cfg["hidden"], cfg["hc"], cfg["ngram_size"], cfg["heads_per_ngram"]
    W, gs, eps = hc * H, cfg["group_size"], cfg["eps"]
    ids = np.asarray(ids, np.int32)
    S = ids.size
    ctx_len = len(context)
    hist = np.concatenate([np.asarray(context, np.int32), ids])
    tw, ts, tb = w["table"]
    rid = ngram_row_ids(hist, ctx_len, n, hpn, w["mult"], w["vocab"], w["offs"], tw.shape[0], cfg["eos"])
    flat = rid.reshape(-1)
    rows = embed_rows(tw, ts, tb, cfg["row_group_size"], np.where(flat < 0, 0, flat))
    rows[flat < 0] = 0
    emb = rows.reshape(S, -1)
    key, _ = qmv(*w["key_proj"], gs, emb)
    value, _ = qmv(*w["value_proj"], gs, emb)
    gated = np.zeros((S, W), np.uint16)
    normed = np.zeros((S, W), np.uint16)
    for t in range(S):
        for c in range(hc):
            sl = slice(c * H, (c + 1) * H)
            gated[t, sl], normed[t, sl], _ = ple_gate(key[t, sl], stream[t, sl], value[t], w["norm_key"][sl],
                                                      w["norm_query"][sl], w["norm_conv"][sl], eps)
    full = np.concatenate([np.asarray(conv_state, np.uint16).reshape(-1, W), normed])
    out = ple_conv(full, w["conv_w"], gated, n)
    total = f32_to_bf16(bf16_to_f32(stream) + bf16_to_f32(out))
    return dict(out=out, sum=total, row_ids=rid, embedded=emb, key=key, value=value, gated=gated, normed=normed,
                full=full, history=hist)


def ple_advance(res, n, nb, ctx_len):
    """The committed PLE state after the first n positions of a window: (conv_state, context)."""
    return res["full"][n:n + nb].copy(), res["history"][n:n + ctx_len].copy()
