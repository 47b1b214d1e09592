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


def download(lw, cfg, lazy=False):
    H, E, F, gs = cfg["hidden"], cfg["experts"], cfg["expert_width"], cfg["group_size"]
    HQ, HK, D, rot, P = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["rot_dims"], cfg["max_positions"]
    QW = lw.qkv_rows

    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(pw, ps, pb, rows, K):
        return (read_device(pw, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(ps, rows * K // gs).reshape(rows, K // gs), bf(pb, rows * K // gs).reshape(rows, K // gs))
    w = dict(attn_norm=bf(lw.attn_norm, H) if lw.attn_norm else None,  # a target's or head's layer has none
             post_norm=bf(lw.post_norm, H) if lw.post_norm else None, q_norm=bf(lw.q_norm, D),
             k_norm=bf(lw.k_norm, D), cos=bf(lw.rope_cos, P * rot).reshape(P, rot),
             sin=bf(lw.rope_sin, P * rot).reshape(P, rot), QW=QW)
    w["qkv"] = q(lw.qkv_w, lw.qkv_s, lw.qkv_b, QW, H)
    w["o"] = q(lw.o_w, lw.o_s, lw.o_b, H, HQ * D)
    w["moe"] = download_moe(lw.moe, cfg, lazy)
    return w


def read_rows(ptr: int, row_bytes: int, r0: int, n: int, out: np.ndarray):
    """Rows r0 .. r0+n-1 of a row-major device array into the same rows of `out`."""
    flat = out.reshape(out.shape[0], -1)
    flat[r0:r0 + n] = read_device(ptr + r0 * row_bytes, n * row_bytes, out.dtype).reshape(n, -1)


class LazyQ4:
    """A q4 matrix whose rows are copied from the device on demand (fetch), into host arrays
    that start as untouched zero pages: a test reads only the rows its tokens use (embedding
    rows, routed experts, n-gram table rows) of matrices of many GB."""

    def __init__(self, q4w, q4s, q4b, rows, K, gs):
        self.ptr = (q4w, q4s, q4b)
        self.K, self.gs = K, gs
        self.arrays = (np.zeros((rows, K // 8), np.uint32), np.zeros((rows, K // gs), np.uint16),
                       np.zeros((rows, K // gs), np.uint16))
        self.have = np.zeros(rows, bool)

    def fetch(self, rows):
        rows = np.unique(np.asarray(rows, np.int64).reshape(-1))
        rows = rows[(rows >= 0) & (rows < self.have.size)]
        for r in rows[~self.have[rows]]:
            for ptr, a in zip(self.ptr, self.arrays):
                read_rows(ptr, a.shape[1] * a.itemsize, int(r), 1, a)
        self.have[rows] = True

    def fetch_range(self, r0, n):
        if not self.have[r0:r0 + n].all():
            for ptr, a in zip(self.ptr, self.arrays):
                read_rows(ptr, a.shape[1] * a.itemsize, r0, n, a)
            self.have[r0:r0 + n] = True


def download_moe(m, cfg, lazy=False):
    """A layer's MoE weights (mtpx_moe_weights) as the dict O.moe_block takes.  lazy: the routed
    experts' rows stay on the device until moe_y fetches the experts a window selects."""
    H, E, F, gs = cfg["hidden"], cfg["experts"], cfg["expert_width"], cfg["group_size"]

    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(pw, ps, pb, rows, K):
        return (read_device(pw, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(ps, rows * K // gs).reshape(rows, K // gs), bf(pb, rows * K // gs).reshape(rows, K // gs))
    moe = dict(router=bf(m.router, E * H).reshape(E, H))
    if m.shared_gate_w:  # the q4 gate row
        moe["sg_w"], moe["sg_s"], moe["sg_b"] = q(m.shared_gate_w, m.shared_gate_s, m.shared_gate_b, 1, H)
    else:
        moe["shared_gate"] = bf(m.shared_gate, H)
    for n, rows, K in (("gate", E * F, H), ("up", E * F, H), ("down", E * H, F),
                       ("sh_gate", F, H), ("sh_up", F, H), ("sh_down", H, F)):
        ptrs = (getattr(m, n + "_w"), getattr(m, n + "_s"), getattr(m, n + "_b"))
        if lazy and not n.startswith("sh_"):
            lq = LazyQ4(*ptrs, rows, K, gs)
            moe["_lazy_" + n] = lq
            moe[n + "_w"], moe[n + "_s"], moe[n + "_b"] = lq.arrays
        else:
            moe[n + "_w"], moe[n + "_s"], moe[n + "_b"] = q(*ptrs, rows, K)
    return moe


def moe_y(moe, x, H, E, K, F, gs):
    """O.moe_block(moe, x)["y"]; with lazily downloaded weights the experts the oracle's own
    router picks for x are fetched first."""
    if "_lazy_gate" in moe:
        xf = O.bf16_to_f32(np.asarray(x, np.uint16).reshape(-1, H))
        picked = set()
        for row in xf:
            idx, _ = O.topk_softmax(O.router_gemv(moe["router"], row[None, :]), K)
            picked.update(int(e) for e in np.asarray(idx).reshape(-1))
        for e in picked:
            moe["_lazy_gate"].fetch_range(e * F, F)
            moe["_lazy_up"].fetch_range(e * F, F)
            moe["_lazy_down"].fetch_range(e * H, H)
    return O.moe_block(moe, x, H, E, K, F, gs)["y"]


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
    m = moe_y(w["moe"], h2, H, cfg["experts"], cfg["top_k"], cfg["expert_width"], gs)
    return O.f32_to_bf16(O.bf16_to_f32(s_) + O.bf16_to_f32(m))
