"""Writes the golden fixtures of tests/test_golden.py (test infrastructure).

The fixtures are outputs of the build's CPU oracle (oracle/) on seeded inputs:
the reference's own outputs for this path cannot be produced here (Swift and
Metal are absent, the MLX CPU build needs LAPACK/CBLAS and network fetches), so
these pin the oracle and the kernels against regressions, beside the
closed-form and brute-force pins of tests/test_oracle_pin.py.  Large inputs
are stored as their recipe (seed and shape; numpy's PCG64 stream is the same
on every platform) plus a SHA-256 of the generated arrays; small inputs are
stored whole.  Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def rand_bf16(r, shape, scale=1.0):
    return O.f32_to_bf16((r.standard_normal(shape) * scale).astype(np.float32))


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# --- config 1: the Qwen3-MoE FFN block (H 2048, 64 experts, top-8 + shared, F 768, gs 64)
C1 = dict(H=2048, E=64, K=8, F=768, gs=64, wseed=0x5EED0001, xseed=0x5EED0002)


def c1_weights(c=C1):
    r = np.random.default_rng(c["wseed"])
    H, E, F, gs = c["H"], c["E"], c["F"], c["gs"]
    w = {"router": rand_bf16(r, (E, H), 0.02), "shared_gate": rand_bf16(r, (H,), 0.02)}
    for name, (rows, k) in {"gate": (E * F, H), "up": (E * F, H), "down": (E * H, F),
                            "sh_gate": (F, H), "sh_up": (F, H), "sh_down": (H, F)}.items():
        w[name + "_w"], w[name + "_s"], w[name + "_b"] = O.affine_quantize(rand_bf16(r, (rows, k), 0.02), gs)
    return w


def c1_x(M, c=C1):
    return rand_bf16(np.random.default_rng(c["xseed"] + M), (M, c["H"]), 1.0)


def c1_fixture():
    w = c1_weights()
    out = {"weights_sha256": np.array(sha(*[w[k] for k in sorted(w)]))}
    for M in (1, 4):
        ref = O.moe_block(w, c1_x(M), C1["H"], C1["E"], C1["K"], C1["F"], C1["gs"])
        out[f"idx_M{M}"] = ref["idx"].astype(np.int32)
        out[f"y_M{M}"] = ref["y"]
    return out


# --- q4 GEMV at small row counts (every depth of the model family, both group sizes)
QMV_CASES = [(K, gs) for K in (256, 640, 768, 2048, 2560) for gs in (32, 64)]


def qmv_inputs(K, gs, N=16, M=2):
    r = np.random.default_rng(K * 100 + gs)
    wq, s, b = O.affine_quantize(rand_bf16(r, (N, K), 0.02), gs)
    return wq, s, b, rand_bf16(r, (M, K), 1.0)


def qmv_fixture():
    out = {}
    for K, gs in QMV_CASES:
        wq, s, b, x = qmv_inputs(K, gs)
        y, yf = O.qmv(wq, s, b, gs, x)
        for name, a in (("wq", wq), ("s", s), ("b", b), ("x", x), ("y", y), ("yf", yf)):
            out[f"K{K}_gs{gs}_{name}"] = a
    return out


# --- config 2: acceptance (V 151936, k in 1/3/5, agreement rate p), greedy and T = 0.7 sampling
C2_V = 151936


def c2_inputs(k, p, seed):
    r = np.random.default_rng(seed)
    t = (r.standard_normal((k + 1, C2_V)) * 2.0).astype(np.float32)
    am = t.argmax(1)
    drafts = np.empty(k, np.int32)
    for i in range(k):
        if r.random() < p:
            drafts[i] = am[i]
        else:
            d = r.integers(0, C2_V - 1)
            drafts[i] = d + (d >= am[i])
    dl = (r.standard_normal((k, C2_V)) * 2.0).astype(np.float32)
    for i in range(k):
        dl[i, drafts[i]] += 6.0
    return t, dl, drafts


C2_CASES = [(k, p, 1000 * k + int(10 * p)) for k in (1, 3, 5) for p in (0.3, 0.6, 0.9)]


def c2_fixture():
    out = {}
    for k, p, seed in C2_CASES:
        t, dl, drafts = c2_inputs(k, p, seed)
        tag = f"k{k}_p{int(10 * p)}"
        out[f"{tag}_sha256"] = np.array(sha(t, dl, drafts))
        out[f"{tag}_greedy"] = np.array(O.accept_greedy(t, drafts, 1024), np.int32)
        out[f"{tag}_sample"] = np.array(O.accept_sample(t, dl, drafts, 0.7, 0xC0FFEE + seed, 7, 2048), np.int32)
    return out


# --- decode/verify attention: T prior positions, S window tokens (8 query heads over 2 KV heads, D 128)
ATT = dict(HQ=8, HK=2, D=128, ROT=32)
ATT_CASES = [(T0, S) for T0 in (1, 33, 1024) for S in (1, 2, 4, 6)]


def att_inputs(T0, S, c=ATT):
    r = np.random.default_rng(7000 + T0 * 10 + S)
    HQ, HK, D = c["HQ"], c["HK"], c["D"]
    tmax = T0 + 8
    QW = 2 * HQ * D + 2 * HK * D + 128
    qkv = rand_bf16(r, (S, QW))
    qn = O.f32_to_bf16((1 + 0.1 * r.standard_normal(D)).astype(np.float32))
    kn = O.f32_to_bf16((1 + 0.1 * r.standard_normal(D)).astype(np.float32))
    kc = rand_bf16(r, (HK, tmax, D))
    vc = rand_bf16(r, (HK, tmax, D))
    return qkv, qn, kn, kc, vc, tmax


def att_oracle(T0, S, c=ATT):
    HQ, HK, D, ROT = c["HQ"], c["HK"], c["D"], c["ROT"]
    qkv, qn, kn, kc, vc, tmax = att_inputs(T0, S)
    cos_t, sin_t = O.rope_table(tmax, ROT, 1e7)
    q_o, k_o, v_o = O.attn_prep(qkv, HQ, HK, D, ROT, qn, kn, 1e-6, cos_t, sin_t, T0)
    kc_o, vc_o = kc.copy(), vc.copy()
    for s in range(S):
        kc_o[:, T0 + s] = k_o[s]
        vc_o[:, T0 + s] = v_o[s]
    att = O.attn_verify(q_o, kc_o, vc_o, T0 + S, np.float32(D ** -0.5), O.ATTN_CHUNK)
    return O.attn_gate(att.reshape(S, HQ * D), qkv, HQ * D)


def att_fixture():
    return {f"T{T0}_S{S}_gated": att_oracle(T0, S) for T0, S in ATT_CASES}


FIXTURES = {"c1_ffn.npz": c1_fixture, "qmv_small.npz": qmv_fixture, "c2_accept.npz": c2_fixture,
            "attention.npz": att_fixture}

if __name__ == "__main__":
    for name, fn in FIXTURES.items():
        np.savez_compressed(os.path.join(HERE, name), **fn())
        print("wrote", name, os.path.getsize(os.path.join(HERE, name)), "bytes")
