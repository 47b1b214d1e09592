"""Pins the CPU oracle independently of the GPU.

Each oracle function is checked against something that does not share its
code: float64 brute force on small inputs, torch's bf16 rounding, libm's exp,
closed forms and hand-computed known answers, the published Philox4x32-10
known-answer vectors, and distributional properties of speculative sampling.
A plausible slip (dropped bias term, wrong nibble order, transposed operand,
off-by-one in the accept prefix) fails at least one of these.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def rng(seed=0):
    return np.random.default_rng(seed)


def bf16(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def f32(h):
    return O.bf16_to_f32(h)


# ---------------------------------------------------------------------------- scalars
def test_bf16_rounding_matches_torch():
    import torch

    r = rng(1)
    x = np.concatenate([
        r.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** r.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.3895314e38, 1e-40], np.float32),
    ]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), want)
    lib = O.lib()
    for v in x[:2000]:
        assert lib.o_f2bf(float(v)) == O.f32_to_bf16(np.array([v], np.float32))[0]


def test_expf_within_2ulp_of_libm():
    xs = np.concatenate([np.linspace(-87.0, 88.5, 40001), rng(2).uniform(-20, 20, 20000)]).astype(np.float32)
    lib = O.lib()
    got = np.array([lib.o_expf(float(v)) for v in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2, ulp.max()
    assert lib.o_expf(0.0) == 1.0
    assert lib.o_expf(-100.0) == 0.0
    assert math.isinf(lib.o_expf(100.0))


def test_sigmoid_silu_bf16_close_to_float64():
    lib = O.lib()
    xs = f32(bf16(np.linspace(-12, 12, 3001)))
    for x in xs:
        s = lib.o_sigmoid_bf16(float(x))
        ref = 1.0 / (1.0 + math.exp(-float(x)))
        # four bf16 roundings (exp, 1+e, 1/d, 1-y): within 4 bf16 ulps
        assert abs(s - ref) <= 2 ** -6 * max(abs(ref), 2 ** -7), (x, s, ref)
        si = lib.o_silu_bf16(float(x))
        assert abs(si - x * ref) <= 2 ** -5 * abs(x * ref) + 1e-6, (x, si)


# ---------------------------------------------------------------------------- a1 quantize
def test_quantize_known_answer():
    # a group of 0, 1/15, ..., 1 (twice): mask false (|min| < |max|), edge = max = 1,
    # scale = (1-0)/15 negated -> q0 = rint(1/scale) = -15, scale = 1/-15, bias = 1,
    # q_j = rint((w_j - 1) / scale) = 15 - j.
    w = np.tile(np.arange(16, dtype=np.float64) / 15.0, 2)
    wb = bf16(w.astype(np.float32)).reshape(1, 32)
    wq, s, b = O.affine_quantize(wb, 32)
    q = ((wq[0][:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(-1)
    wv = f32(wb[0]).astype(np.float64)
    expect_q = np.rint((wv - 1.0) / np.float32(1.0 / -15.0)).clip(0, 15)
    assert np.array_equal(q, expect_q)
    assert np.array_equal(q[:16], 15 - np.arange(16))
    assert f32(b)[0, 0] == 1.0
    assert f32(s)[0, 0] == f32(bf16(np.float32(1.0) / np.float32(-15.0)))


@pytest.mark.parametrize("gs", [32, 64])
def test_quantize_invariants(gs):
    r = rng(3)
    w = bf16(r.standard_normal((64, 256)).astype(np.float32) * 0.02)
    wq, s, b = O.affine_quantize(w, gs)
    deq = O.dequantize(wq, s, b, gs)
    wf = f32(w).astype(np.float64).reshape(64, 256)
    sc = np.repeat(np.abs(f32(s).astype(np.float64)), gs, axis=-1)
    bb = np.repeat(np.abs(f32(b).astype(np.float64)), gs, axis=-1)
    # round trip: within one step (the snapped scale can clip the far end of the
    # range), within half a step for the bulk, plus the bf16 rounding of s and b
    err = np.abs(deq - wf)
    slack = 15 * sc * 2 ** -8 + bb * 2 ** -8 + 1e-12
    assert np.all(err <= sc + slack)
    assert np.mean(err <= 0.5 * sc + slack) > 0.97
    q = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(64, 256)
    assert q.max() <= 15
    # the group's edge value (bf16 already) is stored as the bias and reconstructs exactly
    gsz = wf.reshape(64, -1, gs)
    mx, mn = gsz.max(-1), gsz.min(-1)
    edge = np.where(np.abs(mn) > np.abs(mx), mn, mx)
    assert np.array_equal(f32(b).astype(np.float64), edge)
    # an independent vectorised restatement of the MLX algorithm gives the same bits
    g = wf.reshape(64, -1, gs).astype(np.float32)
    wmax, wmin = g.max(-1), g.min(-1)
    mask = np.abs(wmin) > np.abs(wmax)
    scale = np.maximum((wmax - wmin) / np.float32(15), np.float32(1e-7)).astype(np.float32)
    scale = np.where(mask, scale, -scale).astype(np.float32)
    edge = np.where(mask, wmin, wmax).astype(np.float32)
    q0 = np.rint(edge / scale)
    scale = np.where(q0 != 0, edge / np.where(q0 == 0, 1, q0), scale).astype(np.float32)
    bias = np.where(q0 == 0, 0, edge).astype(np.float32)
    qq = np.clip(np.rint((g - bias[..., None]) / scale[..., None]), 0, 15).astype(np.uint32)
    words = (qq.reshape(64, -1, 8) << (4 * np.arange(8, dtype=np.uint32))).sum(-1).astype(np.uint32)
    assert np.array_equal(words.reshape(wq.shape), wq)
    assert np.array_equal(bf16(scale), s)
    assert np.array_equal(bf16(bias), b)


# ---------------------------------------------------------------------------- a2-a4 GEMV
def test_xblock_is_exact_fixed_point():
    r = rng(4)
    for trial in range(200):
        x = bf16(r.standard_normal(32).astype(np.float32) * np.float32(2.0) ** r.integers(-20, 20, 32))
        m, E = O.xblock(x)
        p = 2.0 ** (E - 149)
        xv = f32(x).astype(np.float64)
        # exact for every element within 2^15 of the block maximum, truncated toward zero below
        big = np.abs(xv) >= np.abs(xv).max() * 2.0 ** -14
        assert np.array_equal(m[big] * p, xv[big])
        assert np.all(np.abs(m * p) <= np.abs(xv))
        assert np.all(np.abs(xv - m * p) < 2.0 ** (E - 149) + 1e-300)
        assert np.abs(m).max() < 2 ** 23


@pytest.mark.parametrize("K,gs,M", [(256, 32, 1), (640, 64, 3), (768, 64, 2), (2048, 32, 1), (96, 32, 4)])
def test_qmv_matches_float64_dequant_matmul(K, gs, M):
    r = rng(K + gs + M)
    N = 48
    w = bf16(r.standard_normal((N, K)).astype(np.float32) * 0.02)
    wq, s, b = O.affine_quantize(w, gs)
    x = bf16(r.standard_normal((M, K)).astype(np.float32))
    y, yf = O.qmv(wq, s, b, gs, x)
    W = O.dequantize(wq, s, b, gs)
    X = f32(x).astype(np.float64)
    ref = X @ W.T
    mag = np.abs(X) @ np.abs(W).T
    assert np.all(np.abs(yf - ref) <= 1e-6 * mag + 1e-30)
    assert np.array_equal(y, bf16(yf))


def test_qmv_rows_are_independent():
    r = rng(7)
    K, gs = 512, 64
    w = bf16(r.standard_normal((40, K)).astype(np.float32) * 0.02)
    wq, s, b = O.affine_quantize(w, gs)
    x = bf16(r.standard_normal((3, K)).astype(np.float32))
    y, _ = O.qmv(wq, s, b, gs, x)
    # row concatenation and per-row M splitting are bit-neutral
    ya, _ = O.qmv(wq[:17], s[:17], b[:17], gs, x)
    yb, _ = O.qmv(wq[17:], s[17:], b[17:], gs, x)
    assert np.array_equal(np.concatenate([ya, yb], 1), y)
    for m in range(3):
        ym, _ = O.qmv(wq, s, b, gs, x[m:m + 1])
        assert np.array_equal(ym[0], y[m])


def test_lanes_rule():
    assert [O.lanes_for_blocks(n) for n in (1, 7, 8, 10, 20, 24, 64, 80, 192, 320, 1000)] == \
        [1, 1, 2, 2, 4, 4, 16, 16, 32, 64, 64]


# ---------------------------------------------------------------------------- router
def test_router_gemv_matches_float64():
    r = rng(8)
    E, H, M = 96, 1024, 3
    W = bf16(r.standard_normal((E, H)).astype(np.float32) * 0.02)
    x = r.standard_normal((M, H)).astype(np.float32)
    out = O.router_gemv(W, x)
    Wf = f32(W).astype(np.float64).reshape(E, H)
    ref = x.astype(np.float64) @ Wf.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(Wf).T
    assert np.all(np.abs(out - ref) <= 2e-6 * mag)


def test_topk_softmax_rule_and_ties():
    r = rng(9)
    lg = r.standard_normal((5, 64)).astype(np.float32)
    lg[0, [3, 7, 9, 40]] = 5.0  # a four-way tie at the top
    lg[1, :] = 1.0              # all equal
    idx, w = O.topk_softmax(lg, 8)
    for m in range(5):
        order = np.lexsort((np.arange(64), -lg[m]))[:8]
        assert np.array_equal(idx[m], order)
        v = lg[m, order].astype(np.float64)
        e = np.exp(v - v.max())
        assert np.allclose(w[m], e / e.sum(), rtol=2e-6, atol=0)
    assert list(idx[0, :4]) == [3, 7, 9, 40]
    assert list(idx[1]) == list(range(8))


def test_topk_nan_ranks_as_minus_inf():
    r = rng(10)
    lg = r.standard_normal((3, 40)).astype(np.float32)
    lg[0, [2, 5, 30]] = np.nan
    lg[1, :] = np.nan               # every logit NaN: the K lowest indices
    lg[2, ::2] = np.nan
    idx, _ = O.topk_softmax(lg, 12)
    for m in range(3):
        clean = np.where(np.isnan(lg[m]), -np.inf, lg[m])
        assert np.array_equal(idx[m], np.lexsort((np.arange(40), -clean))[:12])
        assert len(set(idx[m])) == 12
    assert list(idx[1]) == list(range(12))


# ---------------------------------------------------------------------------- MoE block
def _moe_weights(r, H, E, K, F, gs):
    def q(shape):
        w = bf16(r.standard_normal(shape).astype(np.float32) * 0.02)
        return O.affine_quantize(w, gs)
    gw, gsc, gb = q((E, F, H))
    uw, usc, ub = q((E, F, H))
    dw, dsc, db = q((E, H, F))
    sgw, sgs, sgb = q((F, H))
    suw, sus, sub = q((F, H))
    sdw, sds, sdb = q((H, F))
    return dict(
        router=bf16(r.standard_normal((E, H)).astype(np.float32) * 0.02),
        shared_gate=bf16(r.standard_normal(H).astype(np.float32) * 0.02),
        gate_w=gw, gate_s=gsc, gate_b=gb, up_w=uw, up_s=usc, up_b=ub, down_w=dw, down_s=dsc, down_b=db,
        sh_gate_w=sgw, sh_gate_s=sgs, sh_gate_b=sgb, sh_up_w=suw, sh_up_s=sus, sh_up_b=sub,
        sh_down_w=sdw, sh_down_s=sds, sh_down_b=sdb)


def test_moe_block_matches_float64_textbook():
    H, E, K, F, gs, M = 256, 16, 4, 128, 64, 3
    r = rng(10)
    w = _moe_weights(r, H, E, K, F, gs)
    x = bf16(r.standard_normal((M, H)).astype(np.float32))
    out = O.moe_block(w, x, H, E, K, F, gs)
    X = f32(x).astype(np.float64)
    R = f32(w["router"]).astype(np.float64).reshape(E, H)
    logits = X @ R.T
    assert np.allclose(out["logits"], logits, rtol=0, atol=1e-5)
    G = O.dequantize(w["gate_w"], w["gate_s"], w["gate_b"], gs)
    U = O.dequantize(w["up_w"], w["up_s"], w["up_b"], gs)
    Dn = O.dequantize(w["down_w"], w["down_s"], w["down_b"], gs)
    SG = O.dequantize(w["sh_gate_w"], w["sh_gate_s"], w["sh_gate_b"], gs)
    SU = O.dequantize(w["sh_up_w"], w["sh_up_s"], w["sh_up_b"], gs)
    SD = O.dequantize(w["sh_down_w"], w["sh_down_s"], w["sh_down_b"], gs)
    sgate = f32(w["shared_gate"]).astype(np.float64)
    silu = lambda v: v / (1 + np.exp(-v))
    for m in range(M):
        order = np.argsort(-logits[m], kind="stable")[:K]
        assert np.array_equal(np.sort(out["idx"][m]), np.sort(order))
        v = logits[m, order]
        p = np.exp(v - v.max()); p /= p.sum()
        y = np.zeros(H)
        for k, e in enumerate(order):
            a = silu(G[e] @ X[m]) * (U[e] @ X[m])
            y += p[k] * (Dn[e] @ a)
        a = silu(SG @ X[m]) * (SU @ X[m])
        g = 1 / (1 + np.exp(-(sgate @ X[m])))
        y += g * (SD @ a)
        got = f32(out["y"][m]).astype(np.float64)
        assert np.linalg.norm(got - y) <= 2e-2 * np.linalg.norm(y), np.linalg.norm(got - y) / np.linalg.norm(y)


def test_moe_block_q4_shared_gate():
    """The shared-expert gate as a q4 row (the checkpoint's mlp.shared_expert_gate): the gate is the
    q4 GEMV of that row rounded to bf16 (equal to O.qmv of it, whose arithmetic is pinned above), the
    routing does not depend on it, and the block matches the float64 textbook MoE with the row
    dequantised; with the bf16 row given as well, the q4 row wins."""
    H, E, K, F, gs, M = 256, 16, 4, 128, 32, 3
    r = rng(12)
    w = _moe_weights(r, H, E, K, F, gs)
    sg = bf16(r.standard_normal((1, H)).astype(np.float32) * 0.3)
    w["sg_w"], w["sg_s"], w["sg_b"] = O.affine_quantize(sg, gs)
    x = bf16(r.standard_normal((M, H)).astype(np.float32))
    out = O.moe_block(w, x, H, E, K, F, gs)
    gq, _ = O.qmv(w["sg_w"], w["sg_s"], w["sg_b"], gs, x)
    assert np.array_equal(out["gate"], gq[:, 0])
    base = O.moe_block({k: v for k, v in w.items() if not k.startswith("sg_")}, x, H, E, K, F, gs)
    assert np.array_equal(out["idx"], base["idx"]) and np.array_equal(out["w"], base["w"])
    assert not np.array_equal(out["y"], base["y"])
    X = f32(x).astype(np.float64)
    logits = X @ f32(w["router"]).astype(np.float64).reshape(E, H).T
    G, U, Dn = (O.dequantize(w[n + "_w"], w[n + "_s"], w[n + "_b"], gs) for n in ("gate", "up", "down"))
    SG, SU, SD = (O.dequantize(w[n + "_w"], w[n + "_s"], w[n + "_b"], gs) for n in ("sh_gate", "sh_up", "sh_down"))
    SGT = O.dequantize(w["sg_w"], w["sg_s"], w["sg_b"], gs)[0]
    silu = lambda v: v / (1 + np.exp(-v))
    for m in range(M):
        order = np.argsort(-logits[m], kind="stable")[:K]
        v = logits[m, order]
        p = np.exp(v - v.max()); p /= p.sum()
        y = np.zeros(H)
        for k, e in enumerate(order):
            y += p[k] * (Dn[e] @ (silu(G[e] @ X[m]) * (U[e] @ X[m])))
        y += (SD @ (silu(SG @ X[m]) * (SU @ X[m]))) / (1 + np.exp(-(SGT @ X[m])))
        got = f32(out["y"][m]).astype(np.float64)
        assert np.linalg.norm(got - y) <= 2e-2 * np.linalg.norm(y)
        assert abs(f32(out["gate"][m]) - SGT @ X[m]) <= 1e-2 * abs(SGT @ X[m]) + 1e-3


# ---------------------------------------------------------------------------- attention
def test_rope_table_against_numpy():
    c, s = O.rope_table(64, 16, 1e7)
    half = 8
    i = np.arange(16) % half
    inv = 1e7 ** (-2.0 * i / 16)
    ang = np.arange(64)[:, None] * inv[None, :]
    assert np.max(np.abs(f32(c) - np.cos(ang))) <= 2 ** -8
    assert np.max(np.abs(f32(s) - np.sin(ang))) <= 2 ** -8


def test_attn_prep_matches_float64():
    r = rng(11)
    S, HQ, HK, D, ROT = 3, 4, 2, 64, 16
    QW = 2 * HQ * D + 2 * HK * D + 8
    qkv = bf16(r.standard_normal((S, QW)).astype(np.float32))
    qn = bf16(1 + 0.1 * r.standard_normal(D).astype(np.float32))
    kn = bf16(1 + 0.1 * r.standard_normal(D).astype(np.float32))
    c, s = O.rope_table(32, ROT, 1e7)
    q, k, v = O.attn_prep(qkv, HQ, HK, D, ROT, qn, kn, 1e-6, c, s, 5)
    X = f32(qkv).astype(np.float64)

    def ref(vec, wn, pos):
        y = vec / np.sqrt(np.mean(vec ** 2) + 1e-6) * f32(wn)
        cc, ss = f32(c[pos]).astype(np.float64), f32(s[pos]).astype(np.float64)
        o = y.copy()
        h = ROT // 2
        o[:h] = y[:h] * cc[:h] - y[h:ROT] * ss[:h]
        o[h:ROT] = y[h:ROT] * cc[h:ROT] + y[:h] * ss[h:ROT]
        return o

    for si in range(S):
        for h in range(HQ):
            want = ref(X[si, h * D:(h + 1) * D], qn, 5 + si)
            assert np.max(np.abs(f32(q[si, h]) - want)) <= 3e-2 * np.max(np.abs(want))
        for h in range(HK):
            off = 2 * HQ * D
            want = ref(X[si, off + h * D: off + (h + 1) * D], kn, 5 + si)
            assert np.max(np.abs(f32(k[si, h]) - want)) <= 3e-2 * np.max(np.abs(want))
            assert np.array_equal(v[si, h], qkv[si, off + HK * D + h * D: off + HK * D + (h + 1) * D])


@pytest.mark.parametrize("T,S,chunk", [(1, 1, 32), (33, 2, 32), (70, 4, 16), (40, 6, 64)])
def test_attn_verify_matches_float64(T, S, chunk):
    r = rng(T * 10 + S)
    HQ, HK, D, tmax = 6, 2, 64, 128
    q = bf16(r.standard_normal((S, HQ, D)).astype(np.float32))
    kc = bf16(r.standard_normal((HK, tmax, D)).astype(np.float32))
    vc = bf16(r.standard_normal((HK, tmax, D)).astype(np.float32))
    scale = D ** -0.5
    out = O.attn_verify(q, kc, vc, T, scale, chunk)
    Q, Kf, Vf = (f32(a).astype(np.float64) for a in (q, kc, vc))
    for s in range(S):
        for h in range(HQ):
            hk = h // (HQ // HK)
            last = T - S + s
            sc = Kf[hk, :last + 1] @ Q[s, h] * scale
            p = np.exp(sc - sc.max()); p /= p.sum()
            want = p @ Vf[hk, :last + 1]
            assert np.max(np.abs(f32(out[s, h]) - want)) <= 1e-2 * max(1.0, np.max(np.abs(want)))


def test_attn_gate_closed_form():
    r = rng(12)
    att = bf16(r.standard_normal((2, 32)).astype(np.float32))
    qkv = bf16(r.standard_normal((2, 80)).astype(np.float32))
    out = O.attn_gate(att, qkv, 10)
    g = f32(qkv[:, 10:42]).astype(np.float64)
    want = f32(att) * (1 / (1 + np.exp(-g)))
    assert np.max(np.abs(f32(out) - want)) <= 2 ** -6 * np.max(np.abs(want))


def test_rmsnorm_matches_float64():
    r = rng(13)
    x = bf16(r.standard_normal((3, 640)).astype(np.float32) * 3)
    w = bf16(1 + 0.1 * r.standard_normal(640).astype(np.float32))
    y = O.rmsnorm(x, w, 1e-6)
    X = f32(x).astype(np.float64)
    want = X / np.sqrt(np.mean(X ** 2, axis=1, keepdims=True) + 1e-6) * f32(w)
    assert np.max(np.abs(f32(y) - want)) <= 2 ** -6 * np.max(np.abs(want))


# ---------------------------------------------------------------------------- acceptance
def test_greedy_accept_known_answers():
    V = 10
    def rows(args):
        lg = np.zeros((len(args), V), np.float32)
        for i, a in enumerate(args):
            lg[i, a] = 1.0
        return lg
    # all accepted: n = k, bonus = argmax of the last row
    assert list(O.accept_greedy(rows([1, 2, 3, 4]), [1, 2, 3], 100)) == [3, 4, 104]
    # first rejected: commit a_0
    assert list(O.accept_greedy(rows([1, 2, 3, 4]), [5, 2, 3], 100)) == [0, 1, 101]
    # mid rejection
    assert list(O.accept_greedy(rows([1, 2, 3, 4]), [1, 2, 9], 7)) == [2, 3, 10]
    # ties resolve to the lowest id on the target side
    lg = rows([1, 2])
    lg[0, 6] = 1.0
    assert list(O.accept_greedy(lg, [6], 0)) == [0, 1, 1]
    assert list(O.accept_greedy(lg, [1], 0)) == [1, 2, 2]


def test_philox_known_answer_vectors():
    # Random123 philox4x32_10 known-answer vectors (Salmon et al., SC'11).
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert [int(v) for v in O.philox(ctr, key)] == want


def test_uniform_mapping():
    assert O.uniform(0) == 0.0
    assert O.uniform(0xFFFFFFFF) == 1.0 - 2.0 ** -24
    assert O.uniform(0x80000000) == 0.5


def test_sample_identical_distributions_always_accept():
    r = rng(14)
    V, k = 64, 3
    t = (r.standard_normal((k + 1, V)) * 2).astype(np.float32)
    d = t[:k].copy()
    for off in range(40):
        drafts = r.integers(0, V, k).astype(np.int32)
        out = O.accept_sample(t, d, drafts, 0.7, 1234, off, 50)
        assert out[0] == k and out[2] == 50 + k + 1


def test_sample_disjoint_support_always_rejects():
    V, k = 32, 2
    t = np.full((k + 1, V), -200.0, np.float32)
    t[:, :8] = 0.0  # target mass on ids 0..7
    d = np.full((k, V), -200.0, np.float32)
    d[:, 16:] = 0.0  # draft mass on ids 16..31
    for off in range(30):
        out = O.accept_sample(t, d, np.array([20, 21], np.int32), 0.7, 99, off, 0)
        assert out[0] == 0 and 0 <= out[1] < 8 and out[2] == 1


def test_sample_emits_target_distribution():
    """Speculative sampling is exact: the first emitted token ~ p_target (chi-square)."""
    V, T = 6, 0.7
    r = rng(15)
    t = (r.standard_normal((2, V)) * 1.5).astype(np.float32)
    d = (r.standard_normal((1, V)) * 1.5).astype(np.float32)
    pt = np.exp((t[0] - t[0].max()) / T); pt /= pt.sum()
    pd = np.exp((d[0] - d[0].max()) / T); pd /= pd.sum()
    counts = np.zeros(V)
    n = 6000
    dr = r.choice(V, size=n, p=pd).astype(np.int32)
    for i in range(n):
        out = O.accept_sample(t, d, dr[i:i + 1], T, 777, i, 0)
        first = dr[i] if out[0] == 1 else out[1]
        counts[first] += 1
    chi2 = ((counts - n * pt) ** 2 / (n * pt)).sum()
    assert chi2 < 25.0, (chi2, counts, n * pt)  # 5 dof, p ~ 1e-4


def test_sample_onehot_drafts_emit_target_distribution():
    """One-hot draft distributions (a greedy drafter, dlogits None): the draft d is accepted with
    probability p_t(d) and a rejection samples p_t without d, so the first emitted token is still
    ~ p_target whatever the draft (chi-square, drafts cycling over every id); and the one-hot rule
    equals the general rule given a draft row whose softmax is one-hot (logit gap of 1000)."""
    V, T = 6, 0.7
    r = rng(19)
    t = (r.standard_normal((2, V)) * 1.5).astype(np.float32)
    pt = np.exp((t[0] - t[0].max()) / T); pt /= pt.sum()
    counts = np.zeros(V)
    acc = np.zeros(V)
    n = 6000
    for i in range(n):
        d = np.array([i % V], np.int32)
        out = O.accept_sample(t, None, d, T, 4242, i, 0)
        first = d[0] if out[0] == 1 else out[1]
        if out[0] == 1:
            acc[d[0]] += 1
        else:
            assert out[1] != d[0]  # a rejected draft is never the resample
        counts[first] += 1
    chi2 = ((counts - n * pt) ** 2 / (n * pt)).sum()
    assert chi2 < 25.0, (chi2, counts, n * pt)
    # acceptance rate of draft v = p_t(v) (each id drafted n / V times)
    assert np.all(np.abs(acc / (n / V) - pt) < 5 * np.sqrt(pt * (1 - pt) / (n / V)) + 1e-9)
    for i in range(200):
        d = np.array([i % V, (i * 7) % V], np.int32)
        t3 = (r.standard_normal((3, V)) * 1.5).astype(np.float32)
        onehot = np.zeros((2, V), np.float32)
        onehot[0, d[0]] = onehot[1, d[1]] = 1000.0
        assert list(O.accept_sample(t3, None, d, T, 99, i, 5)) == list(O.accept_sample(t3, onehot, d, T, 99, i, 5))


def test_softmax_row_sum_close_to_fsum():
    e = rng(16).random(151936).astype(np.float32)
    assert abs(O.softmax_row_sum(e) - math.fsum(e.astype(np.float64))) <= 1e-6 * e.sum()


def test_argmax_nan_rule_matches_mlx():
    """MLX's argmax (arg_reduce.metal:42-62): start at (index 0, -inf), take a value only when it is
    strictly greater.  Restated independently as numpy's first-maximum argmax over the row with
    every NaN replaced by -inf; known answers for the NaN / -inf corners."""
    x = np.array([[1.0, np.nan, 3.0, np.nan], [np.nan] * 4, [-np.inf] * 4, [2.0, 5.0, 5.0, -1.0],
                  [np.nan, -np.inf, -np.inf, -np.inf], [-np.inf, np.nan, -5.0, -5.0], [np.nan, 7.0, np.inf, np.inf]],
                 np.float32)
    got = O.argmax_rows(x)
    assert list(got) == [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in x] == [2, 0, 0, 1, 0, 2, 2]
    big = rng(17).standard_normal((3, 5000)).astype(np.float32)
    big[0, rng(18).integers(0, 5000, 400)] = np.nan
    big[1, :] = np.nan
    big[2, 4999] = np.nan
    assert list(O.argmax_rows(big)) == [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in big]
    out = O.accept_greedy(x[1:3].copy(), np.array([0], np.int32), 10)
    assert list(out) == [1, 0, 12]  # row 0 all NaN: argmax 0 == draft 0 accepted; bonus row 1 -> 0


def _top2_lexsort(x):
    """Independent restatement: sort each row by (value desc with NaN as -inf, index asc)."""
    ids, vals = [], []
    for r in x:
        v = np.where(np.isnan(r), -np.inf, r)
        order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))
        ids.append(order[:2])
        vals.append(v[order[:2]])
    return np.array(ids, np.int32), np.array(vals, np.float32)


def test_top2_rows_matches_lexsort():
    """Top two per row against a lexsort of (value desc, index asc), with ties (equal leaders, equal
    runners-up), NaNs, infinities and rows of only NaN / -inf; the first id is the argmax."""
    r = rng(21)
    x = r.standard_normal((12, 3000)).astype(np.float32)
    x[0, [5, 900]] = 9.0                       # tied leaders: 5 then 900
    x[1, 17] = 9.0; x[1, [40, 2999]] = 8.0     # tied runners-up: 40
    x[2, :] = np.nan
    x[3, :] = -np.inf
    x[4, ::3] = np.nan
    x[5, 7] = np.inf; x[5, 8] = np.nan
    x[6] = np.round(x[6])                      # many exact ties
    x[7, :] = 0.0
    got_i, got_v = O.top2_rows(x)
    want_i, want_v = _top2_lexsort(x)
    assert np.array_equal(got_i, want_i) and np.array_equal(got_v, want_v)
    assert list(got_i[:, 0]) == list(O.argmax_rows(x))
    assert list(got_i[0]) == [5, 900] and list(got_i[1]) == [17, 40] and list(got_i[2]) == [0, 1]


# ---------------------------------------------------------------------------- mlx_cpu mode (o_qmm_t_bf16)
def _pack_q(q):
    """q uint8 [N, K] in [0, 15] -> MLX 4-bit words [N, K/8] (element k at bits 4*(k%8))."""
    q = np.asarray(q, np.uint32)
    N, K = q.shape
    w = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        w |= q[:, j::8] << np.uint32(4 * j)
    return w


def test_qmm_t_bf16_integer_dot_is_exact():
    """Integer scales, biases, nibbles and activations whose running sums stay within 256 in
    magnitude: every bf16 rounding of MLX's _qmm_t is exact, so the result is the integer dot of
    the dequantised rows.  Four groups of 32 with different (scale, bias) and a 2 x 3 output pin
    the nibble order, the group indexing and the operand roles."""
    r = rng(41)
    M, N, K, gs = 2, 3, 128, 32
    q = r.integers(0, 16, (N, K))
    s = r.choice([1.0, 2.0], (N, K // gs)).astype(np.float32)
    b = r.choice([-8.0, -4.0, 0.0, 3.0], (N, K // gs)).astype(np.float32)
    wdq = np.repeat(s, gs, 1) * q + np.repeat(b, gs, 1)
    while True:
        x = (r.integers(-1, 2, (M, K)) * (r.random((M, K)) < 0.15)).astype(np.float32)
        run = np.cumsum(x[:, None, :] * wdq[None, :, :], axis=2)
        if np.abs(run).max() <= 256 and np.abs(run[..., -1]).min() > 0:
            break
    got = f32(O.qmm_t_bf16(_pack_q(q), bf16(s), bf16(b), gs, bf16(x)))
    assert np.array_equal(got, x @ wdq.T)


def test_qmm_t_bf16_running_sum_saturates_in_bf16():
    """256 then +1 per element: in bf16, 256 + 1 = 257 rounds (to even) back to 256, so MLX's bf16
    running sum stays at 256; a float accumulation would return 256 + 31 = 287."""
    gs, K = 32, 32
    q = np.zeros((1, K), np.int64)
    q[0, 0] = 15  # w = 1*15 + 1 = 16 at element 0, w = 1 elsewhere
    x = np.ones((1, K), np.float32)
    x[0, 0] = 16.0
    got = f32(O.qmm_t_bf16(_pack_q(q), bf16([[1.0]]), bf16([[1.0]]), gs, bf16(x)))
    assert got[0, 0] == 256.0
    # the same terms in the other order: 31 ones reach 31 exactly, then + 256 = 287 -> bf16 288
    q2, x2 = q[:, ::-1].copy(), x[:, ::-1].copy()
    got2 = f32(O.qmm_t_bf16(_pack_q(q2), bf16([[1.0]]), bf16([[1.0]]), gs, bf16(x2)))
    assert got2[0, 0] == 288.0


def test_qmm_t_bf16_matches_torch_bf16_ops_and_float64_bound():
    """Random operands: equal to the same sequence of operations in torch's own bf16 arithmetic
    (each op computed in float and rounded to bf16 by torch, an implementation independent of the
    oracle's rounding), and within the bf16 accumulation bound of the float64 dot:
    |err| <= (K + 2) * 2^-8 * sum |x * w|."""
    import torch

    r = rng(42)
    M, N, K, gs = 3, 5, 128, 64
    q = r.integers(0, 16, (N, K))
    s = bf16(r.uniform(0.001, 0.02, (N, K // gs)))
    b = bf16(r.uniform(-0.1, 0.0, (N, K // gs)))
    x = bf16(r.standard_normal((M, K)))
    got = f32(O.qmm_t_bf16(_pack_q(q), s, b, gs, x))

    def tb(a):
        return torch.from_numpy(np.ascontiguousarray(f32(a))).to(torch.bfloat16)

    st, bt, xt = tb(s), tb(b), tb(x)
    qt = torch.from_numpy(q.astype(np.float32)).to(torch.bfloat16)
    w = st.repeat_interleave(gs, 1) * qt + bt.repeat_interleave(gs, 1)  # bf16 ops: rounded each
    acc = torch.zeros(M, N, dtype=torch.bfloat16)
    for k in range(K):
        acc = acc + xt[:, k:k + 1] * w[None, :, k]
    assert np.array_equal(got, acc.float().numpy())
    wf = w.double().numpy()
    xf = f32(x).astype(np.float64)
    exact = xf @ wf.T
    bound = (K + 2) * 2.0 ** -8 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(got - exact) <= bound)
