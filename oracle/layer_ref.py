"""Oracle-side composition of one decoder layer -- TEST INFRASTRUCTURE ONLY.

Used by tests/test_gpu_layer.py (parity) and bench.py's cpu_baseline leg
(timing): downloads a layer's device weights and runs the same step through the
CPU oracle.
"""
import ctypes as C

import numpy as np

from oracle import oracle as O

_hip = None


def read_device(ptr: int, nbytes: int, dtype) -> np.ndarray:
    """Copy raw device memory (a pointer the library owns) to the host."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    assert _hip.hipDeviceSynchronize() == 0
    rc = _hip.hipMemcpy(out.ctypes.data, C.c_void_p(ptr), nbytes, 2)  # device -> host
    assert rc == 0, rc
    return out


def download(lw, cfg):
    H, E, F, gs = cfg["hidden"], cfg["experts"], cfg["expert_width"], cfg["group_size"]
    HQ, HK, D, rot, P = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["rot_dims"], cfg["max_positions"]
    QW = lw.qkv_rows

    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(pw, ps, pb, rows, K):
        return (read_device(pw, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(ps, rows * K // gs).reshape(rows, K // gs), bf(pb, rows * K // gs).reshape(rows, K // gs))
    w = dict(attn_norm=bf(lw.attn_norm, H), post_norm=bf(lw.post_norm, H), q_norm=bf(lw.q_norm, D),
             k_norm=bf(lw.k_norm, D), cos=bf(lw.rope_cos, P * rot).reshape(P, rot),
             sin=bf(lw.rope_sin, P * rot).reshape(P, rot), QW=QW)
    w["qkv"] = q(lw.qkv_w, lw.qkv_s, lw.qkv_b, QW, H)
    w["o"] = q(lw.o_w, lw.o_s, lw.o_b, H, HQ * D)
    w["moe"] = download_moe(lw.moe, cfg)
    return w


def download_moe(m, cfg):
    """A layer's MoE weights (mtpx_moe_weights) as the dict O.moe_block takes."""
    H, E, F, gs = cfg["hidden"], cfg["experts"], cfg["expert_width"], cfg["group_size"]

    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(pw, ps, pb, rows, K):
        return (read_device(pw, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(ps, rows * K // gs).reshape(rows, K // gs), bf(pb, rows * K // gs).reshape(rows, K // gs))
    moe = dict(router=bf(m.router, E * H).reshape(E, H), shared_gate=bf(m.shared_gate, H))
    for n, rows, K in (("gate", E * F, H), ("up", E * F, H), ("down", E * H, F),
                       ("sh_gate", F, H), ("sh_up", F, H), ("sh_down", H, F)):
        moe[n + "_w"], moe[n + "_s"], moe[n + "_b"] = q(getattr(m, n + "_w"), getattr(m, n + "_s"),
                                                         getattr(m, n + "_b"), rows, K)
    return moe


def oracle_attn(w, cfg, kc, vc, h, pos0):
    """Attention sublayer on the (already normalised) input h: qkv, prep + KV append,
    verify attention with the output gate, o_proj."""
    HQ, HK, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    gs, eps, S = cfg["group_size"], cfg["eps"], h.shape[0]
    qkv, _ = O.qmv(*w["qkv"], gs, h)
    q, k, v = O.attn_prep(qkv, HQ, HK, D, cfg["rot_dims"], w["q_norm"], w["k_norm"], eps, w["cos"], w["sin"], pos0)
    for s in range(S):
        kc[:, pos0 + s] = k[s]
        vc[:, pos0 + s] = v[s]
    att = O.attn_verify(q, kc, vc, pos0 + S, np.float32(1.0) / np.sqrt(np.float32(D)), O.ATTN_CHUNK)
    g = O.attn_gate(att.reshape(S, HQ * D), qkv, HQ * D)
    o, _ = O.qmv(*w["o"], gs, g)
    return o


def oracle_layer(w, cfg, kc, vc, x, pos0):
    H, gs, eps = cfg["hidden"], cfg["group_size"], cfg["eps"]
    h1 = O.rmsnorm(x, w["attn_norm"], eps)
    o = oracle_attn(w, cfg, kc, vc, h1, pos0)
    s_ = O.f32_to_bf16(O.bf16_to_f32(x) + O.bf16_to_f32(o))
    h2 = O.rmsnorm(s_, w["post_norm"], eps)
    m = O.moe_block(w["moe"], h2, H, cfg["experts"], cfg["top_k"], cfg["expert_width"], gs)["y"]
    return O.f32_to_bf16(O.bf16_to_f32(s_) + O.bf16_to_f32(m))
