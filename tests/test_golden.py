"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py): the
oracle must reproduce them on the CPU, and the HIP kernels through the C ABI
on the GPU, bit for bit.  Inputs are regenerated from their recipes (numpy
PCG64 seeds); a SHA-256 of each regenerated input guards the recipe itself.
Cases follow BASELINE config 1 (the MoE FFN block at M = 1 and 4), config 2
(greedy and T = 0.7 acceptance over V = 151936, k in 1/3/5, p in .3/.6/.9), the
q4 GEMV at every depth of the family with both group sizes, and decode/verify
attention at T in 1/33/1024 prior positions and S in 1/2/4/6 window tokens."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as G  # noqa: E402
from oracle import oracle as O  # noqa: E402


def load(name):
    return np.load(os.path.join(HERE, "golden", name), allow_pickle=False)


# ---------------------------------------------------------------------------- CPU: the oracle
def test_golden_qmv_oracle():
    f = load("qmv_small.npz")
    for K, gs in G.QMV_CASES:
        wq, s, b, x = G.qmv_inputs(K, gs)
        for name, a in (("wq", wq), ("s", s), ("b", b), ("x", x)):
            assert np.array_equal(a, f[f"K{K}_gs{gs}_{name}"]), (K, gs, name)
        y, yf = O.qmv(wq, s, b, gs, x)
        assert np.array_equal(y, f[f"K{K}_gs{gs}_y"])
        assert np.array_equal(yf.view(np.uint32), f[f"K{K}_gs{gs}_yf"].view(np.uint32))


def test_golden_attention_oracle():
    f = load("attention.npz")
    for T0, S in G.ATT_CASES:
        assert np.array_equal(G.att_oracle(T0, S), f[f"T{T0}_S{S}_gated"]), (T0, S)


def test_golden_accept_oracle():
    f = load("c2_accept.npz")
    for k, p, seed in G.C2_CASES:
        t, dl, drafts = G.c2_inputs(k, p, seed)
        tag = f"k{k}_p{int(10 * p)}"
        assert G.sha(t, dl, drafts) == str(f[f"{tag}_sha256"])
        assert list(O.accept_greedy(t, drafts, 1024)) == list(f[f"{tag}_greedy"])
        assert list(O.accept_sample(t, dl, drafts, 0.7, 0xC0FFEE + seed, 7, 2048)) == list(f[f"{tag}_sample"])


@pytest.fixture(scope="module")
def c1_weights():
    return G.c1_weights()


def test_golden_c1_ffn_oracle(c1_weights):
    f = load("c1_ffn.npz")
    w = c1_weights
    assert G.sha(*[w[k] for k in sorted(w)]) == str(f["weights_sha256"])
    for M in (1, 4):
        ref = O.moe_block(w, G.c1_x(M), G.C1["H"], G.C1["E"], G.C1["K"], G.C1["F"], G.C1["gs"])
        assert np.array_equal(ref["idx"].astype(np.int32), f[f"idx_M{M}"])
        assert np.array_equal(ref["y"], f[f"y_M{M}"])


# ---------------------------------------------------------------------------- GPU: the kernels
@pytest.fixture(scope="module")
def ctx():
    from gpu_util import need_gpu
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


@pytest.mark.gpu
def test_golden_qmv_gpu(ctx):
    import torch
    from gpu_util import dev, empty_bf16, host
    f = load("qmv_small.npz")
    for K, gs in G.QMV_CASES:
        g = {n: f[f"K{K}_gs{gs}_{n}"] for n in ("wq", "s", "b", "x", "y", "yf")}
        M, N = g["x"].shape[0], g["wq"].shape[0]
        ds, db = dev(g["s"]), dev(g["b"])
        for sb in (None, ctx.pack_sb(ds, db, K, gs)):
            y = empty_bf16(M, N)
            yf = torch.zeros(M, N, dtype=torch.float32, device="cuda")
            ctx.qmv(dev(g["wq"]), ds, db, gs, dev(g["x"]), y, yf, sb=sb)
            ctx.synchronize()
            assert np.array_equal(host(y), g["y"]), (K, gs)
            assert np.array_equal(host(yf).view(np.uint32), g["yf"].view(np.uint32)), (K, gs)


@pytest.mark.gpu
def test_golden_attention_gpu(ctx):
    from gpu_util import dev, empty_bf16, host
    f = load("attention.npz")
    c = G.ATT
    HQ, HK, D, ROT = c["HQ"], c["HK"], c["D"], c["ROT"]
    for T0, S in G.ATT_CASES:
        print("case golden attention", T0, S, flush=True)
        qkv, qn, kn, kc, vc, tmax = G.att_inputs(T0, S)
        cos_t, sin_t = O.rope_table(tmax, ROT, 1e7)
        q = empty_bf16(S, HQ, D)
        kcd, vcd = dev(kc), dev(vc)
        ctx.attn_prep(dev(qkv), HQ, HK, D, ROT, dev(qn), dev(kn), 1e-6, dev(cos_t), dev(sin_t), T0, q, kcd, vcd)
        out = empty_bf16(S, HQ, D)
        gated = empty_bf16(S, HQ * D)
        ctx.attn_verify(q, kcd, vcd, T0 + S, float(np.float32(D ** -0.5)), out=out, qkv=dev(qkv), gate_off=HQ * D,
                        out_gated=gated)
        ctx.synchronize()
        assert np.array_equal(host(gated), f[f"T{T0}_S{S}_gated"]), (T0, S)


@pytest.mark.gpu
def test_golden_accept_gpu(ctx):
    import torch
    from gpu_util import dev, host
    f = load("c2_accept.npz")
    for k, p, seed in G.C2_CASES:
        t, dl, drafts = G.c2_inputs(k, p, seed)
        tag = f"k{k}_p{int(10 * p)}"
        out = torch.zeros(3, dtype=torch.int32, device="cuda")
        ctx.accept_greedy(dev(t), dev(drafts), 1024, out)
        ctx.synchronize()
        assert list(host(out)) == list(f[f"{tag}_greedy"]), tag
        ctx.accept_sample(dev(t), dev(dl), dev(drafts), 0.7, 0xC0FFEE + seed, 7, 2048, out)
        ctx.synchronize()
        assert list(host(out)) == list(f[f"{tag}_sample"]), tag


@pytest.mark.gpu
def test_golden_c1_ffn_gpu(ctx, c1_weights):
    import torch
    import mtpx
    from gpu_util import dev, empty_bf16, host
    f = load("c1_ffn.npz")
    c = G.C1
    dw = {n: dev(v) for n, v in c1_weights.items()}
    for packed in (False, True):
        d = dict(dw)
        if packed:
            for n, Kd in (("gate", c["H"]), ("up", c["H"]), ("down", c["F"]), ("sh_gate", c["H"]), ("sh_up", c["H"]),
                          ("sh_down", c["F"])):
                d[n + "_sb"] = ctx.pack_sb(d[n + "_s"], d[n + "_b"], Kd, c["gs"])
        mw = mtpx.moe_weights_from(d, c["H"], c["E"], c["K"], c["F"], c["gs"])
        for M in (1, 4):
            y = empty_bf16(M, c["H"])
            idx = torch.zeros(M, c["K"], dtype=torch.int32, device="cuda")
            ctx.moe_forward(mw, dev(G.c1_x(M)), y, idx)
            ctx.synchronize()
            assert np.array_equal(host(idx), f[f"idx_M{M}"]), (packed, M)
            assert np.array_equal(host(y), f[f"y_M{M}"]), (packed, M)
