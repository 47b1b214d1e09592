"""GPU parity of verify attention (prep + KV append, split-KV verify, gate) and of
the acceptance kernels (greedy and temperature rejection sampling) against the
oracle, bit-exact.  Acceptance follows config 2 of BASELINE.json: vocab 151936,
k in {1, 3, 5}, fp32 logits N(0, 4), drafts matching the target argmax at rate p."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


# ---------------------------------------------------------------------------- a13-a15
@pytest.mark.parametrize("S,T0,HQ,HK,D,ROT", [
    (1, 1024, 24, 2, 256, 64), (2, 1024, 24, 2, 256, 64), (4, 1024, 24, 2, 256, 64),
    (6, 1024, 24, 2, 256, 64), (1, 0, 24, 2, 256, 64), (3, 31, 8, 2, 64, 16), (5, 65, 4, 4, 128, 32),
])
def test_attention_bit_exact(ctx, S, T0, HQ, HK, D, ROT):
    print("case attn", S, T0, HQ, HK, D, ROT, flush=True)
    r = np.random.default_rng(S * 1000 + T0)
    tmax = T0 + 16
    QW = 2 * HQ * D + 2 * HK * D + 128
    qkv = rand_bf16(r, (S, QW))
    qn = O.f32_to_bf16((1 + 0.1 * r.standard_normal(D)).astype(np.float32))
    kn = O.f32_to_bf16((1 + 0.1 * r.standard_normal(D)).astype(np.float32))
    cos_t, sin_t = O.rope_table(tmax, ROT, 1e7)
    kc = rand_bf16(r, (HK, tmax, D))
    vc = rand_bf16(r, (HK, tmax, D))
    # oracle: prep, append, verify, gate
    q_o, k_o, v_o = O.attn_prep(qkv, HQ, HK, D, ROT, qn, kn, 1e-6, cos_t, sin_t, T0)
    kc_o, vc_o = kc.copy(), vc.copy()
    for s in range(S):
        kc_o[:, T0 + s] = k_o[s]
        vc_o[:, T0 + s] = v_o[s]
    T = T0 + S
    scale = D ** -0.5
    att_o = O.attn_verify(q_o, kc_o, vc_o, T, np.float32(scale), O.ATTN_CHUNK)
    gated_o = O.attn_gate(att_o.reshape(S, HQ * D), qkv, HQ * D)
    # device
    q = empty_bf16(S, HQ, D)
    kcd, vcd = dev(kc), dev(vc)
    ctx.attn_prep(dev(qkv), HQ, HK, D, ROT, dev(qn), dev(kn), 1e-6, dev(cos_t), dev(sin_t), T0, q, kcd, vcd)
    out = empty_bf16(S, HQ, D)
    gated = empty_bf16(S, HQ * D)
    ctx.attn_verify(q, kcd, vcd, T, float(np.float32(scale)), out=out, qkv=dev(qkv), gate_off=HQ * D,
                    out_gated=gated)
    ctx.synchronize()
    assert np.array_equal(host(q), q_o)
    assert np.array_equal(host(kcd), kc_o)
    assert np.array_equal(host(vcd), vc_o)
    assert np.array_equal(host(out), att_o)
    assert np.array_equal(host(gated), gated_o)


def test_kv_rollback_equals_never_advanced(ctx):
    """Rewinding the offset and re-appending gives the cache and the attention a
    window that never advanced would have (docs/qwen38-125b-a6b-port-notes.md:338-343)."""
    import mtpx
    HQ, HK, D, ROT, tmax = 8, 2, 64, 16, 64
    QW = 2 * HQ * D + 2 * HK * D
    r = np.random.default_rng(3)
    cos_t, sin_t = (dev(a) for a in O.rope_table(tmax, ROT, 1e7))
    qn = dev(O.f32_to_bf16(np.ones(D, np.float32)))
    prompt, spec, nxt = (dev(rand_bf16(r, (n, QW))) for n in (8, 4, 2))

    def run(steps):
        kv = mtpx.KVCache(ctx, HK, D, tmax)
        kp, vp, _ = kv.buffers()
        outs = []
        for kind, rows in steps:
            if kind == "trim":
                assert kv.trim(rows) == rows
                continue
            S = rows.shape[0]
            q = empty_bf16(S, HQ, D)
            ctx.attn_prep(rows, HQ, HK, D, ROT, qn, qn, 1e-6, cos_t, sin_t, kv.offset, q, kp, vp, tmax=tmax)
            T = kv.offset + S
            out = empty_bf16(S, HQ, D)
            ctx.attn_verify(q, kp, vp, T, D ** -0.5, out=out, HK=HK, tmax=tmax)
            kv.offset = T
            ctx.synchronize()
            outs.append(host(out))
        return outs, kv

    a, kva = run([("f", prompt), ("f", spec), ("trim", 3), ("f", nxt)])
    b, kvb = run([("f", prompt), ("f", spec[:1]), ("f", nxt)])
    assert kva.offset == kvb.offset == 8 + 1 + 2
    assert np.array_equal(a[0], b[0])
    assert np.array_equal(a[-1], b[-1])


# ---------------------------------------------------------------------------- a18, a21, a22
def c2_case(V, k, p, seed):
    r = np.random.default_rng(seed)
    t = (r.standard_normal((k + 1, V)) * 2.0).astype(np.float32)
    am = t.argmax(1)
    drafts = np.empty(k, np.int32)
    for i in range(k):
        if r.random() < p:
            drafts[i] = am[i]
        else:
            d = r.integers(0, V - 1)
            drafts[i] = d + (d >= am[i])
    dl = (r.standard_normal((k, V)) * 2.0).astype(np.float32)
    # make the draft distribution favour its own proposal, like a real head's
    for i in range(k):
        dl[i, drafts[i]] += 6.0
    return t, dl, drafts


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("p", [0.3, 0.6, 0.9])
def test_accept_greedy_bit_exact(ctx, k, p):
    print("case greedy", k, p, flush=True)
    V = 151936
    for seed in range(4):
        t, _, drafts = c2_case(V, k, p, 100 * k + int(10 * p) + seed)
        want = O.accept_greedy(t, drafts, 1024)
        out = torch.zeros(3, dtype=torch.int32, device="cuda")
        ctx.accept_greedy(dev(t), dev(drafts), 1024, out)
        ctx.synchronize()
        assert list(host(out)) == list(want)


def test_accept_greedy_ties_and_extremes(ctx):
    V = 151936
    t = np.zeros((4, V), np.float32)
    t[0, [5, 70000]] = 3.0     # tie -> 5
    t[1, [V - 1, 9]] = 2.0     # tie -> 9
    t[2, 0] = 1.0
    t[3, V - 1] = 7.0
    for drafts, want in (([5, 9, 0], [3, V - 1, 1028]), ([70000, 9, 0], [0, 5, 1025]), ([5, 9, 1], [2, 0, 1027])):
        out = torch.zeros(3, dtype=torch.int32, device="cuda")
        ctx.accept_greedy(dev(t), dev(np.array(drafts, np.int32)), 1024, out)
        ctx.synchronize()
        assert list(host(out)) == want
        assert list(O.accept_greedy(t, np.array(drafts, np.int32), 1024)) == want


def test_argmax_rows_bit_exact(ctx):
    r = np.random.default_rng(4)
    x = r.standard_normal((7, 248320)).astype(np.float32)
    x[3, 1000] = x[3, 200000] = 100.0
    out = torch.zeros(7, dtype=torch.int32, device="cuda")
    ctx.argmax_rows(dev(x), out)
    ctx.synchronize()
    assert list(host(out)) == list(O.argmax_rows(x))
    assert host(out)[3] == 1000


def test_argmax_and_accept_nan_rows(ctx):
    """MLX's argmax rule: a NaN never wins (it ranks as -inf), an all-NaN row gives id 0, and NaNs
    spread over several of the partial pass's slices do not disturb the winner of another slice."""
    V = 151936
    x = np.random.default_rng(5).standard_normal((4, V)).astype(np.float32)
    x[0, :] = np.nan
    x[1, [70000, 150000]] = np.nan
    x[2, 9] = np.inf
    x[3, 100000] = np.nan
    x[3, 5] = np.inf
    out = torch.zeros(4, dtype=torch.int32, device="cuda")
    ctx.argmax_rows(dev(x), out)
    ctx.synchronize()
    want = [int(np.argmax(np.where(np.isnan(r), -np.inf, r))) for r in x]
    assert want[0] == 0 and want[2] == 9 and want[3] == 5 and want[1] not in (70000, 150000)
    assert list(host(out)) == want == list(O.argmax_rows(x))
    out3 = torch.zeros(3, dtype=torch.int32, device="cuda")
    drafts = np.array([0, want[1], 9], np.int32)
    ctx.accept_greedy(dev(x), dev(drafts), 100, out3)
    ctx.synchronize()
    assert list(host(out3)) == list(O.accept_greedy(x, drafts, 100)) == [3, 5, 104]


@pytest.mark.parametrize("V", [151936, 248320, 2])
def test_top_two_bit_exact(ctx, V):
    """The top-two query (cbv2MTPTopTwo) on f32 logits and on bf16 logits (many exact ties after the
    rounding) against the oracle: ids and values bit-exact, NaN rows and ties included."""
    print("case top two", V, flush=True)
    r = np.random.default_rng(V)
    x = (r.standard_normal((6, V)) * 2.0).astype(np.float32)
    if V > 2:
        x[0, [3, V - 1]] = 50.0
        x[1, :] = np.nan
        x[2, 1::2] = np.nan
        x[3, 100000 % V] = np.inf
    for bf in (False, True):
        xs = O.f32_to_bf16(x) if bf else x
        ids = torch.full((6, 2), -1, dtype=torch.int32, device="cuda")
        vals = torch.zeros(6, 2, dtype=torch.float32, device="cuda")
        ctx.top_two(dev(xs), ids, vals)
        wi, wv = O.top2_rows(O.bf16_to_f32(xs) if bf else x)
        assert np.array_equal(host(ids), wi), bf
        assert np.array_equal(host(vals).view(np.uint32), wv.view(np.uint32)), bf
        if V > 2:
            assert list(wi[0]) == [3, V - 1]


@pytest.mark.parametrize("k", [0, 1, 3, 5])
@pytest.mark.parametrize("p", [0.3, 0.9])
def test_accept_sample_onehot_bit_exact(ctx, k, p):
    """One-hot draft distributions (no draft logits: a greedy drafter) on f32 logits and on their
    bf16 roundings (the verify's output, with the committed tokens): bit-exact against the oracle
    given the same values.  Drafts at the target argmax are accepted with probability p_t."""
    print("case sample onehot", k, p, flush=True)
    V = 151936
    for seed in range(3):
        t, _, drafts = c2_case(V, max(k, 1), p, 700 + 10 * k + int(10 * p) + seed)
        t, drafts = t[:k + 1], drafts[:k]
        tb = O.f32_to_bf16(t)
        for off in (0, 4321):
            for T in (0.7, 0.2):
                want = O.accept_sample(t, None, drafts, T, 0xBEEF + seed, off, 512)
                out = torch.zeros(3, dtype=torch.int32, device="cuda")
                ctx.accept_sample(dev(t), None, dev(drafts), T, 0xBEEF + seed, off, 512, out)
                assert list(host(out)) == list(want), ("f32", seed, off, T)
                want = O.accept_sample(O.bf16_to_f32(tb), None, drafts, T, 0xBEEF + seed, off, 512)
                toks = torch.full((k + 1,), -1, dtype=torch.int32, device="cuda")
                ctx.accept_sample_bf16(dev(tb), None, dev(drafts), T, 0xBEEF + seed, off, 512, out, toks)
                assert list(host(out)) == list(want), ("bf16", seed, off, T)
                n = int(want[0])
                assert list(host(toks))[:n + 1] == list(drafts[:n]) + [int(want[1])]


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("p", [0.3, 0.9])
def test_accept_sample_bit_exact(ctx, k, p):
    print("case sample", k, p, flush=True)
    V = 151936
    for seed in range(3):
        t, dl, drafts = c2_case(V, k, p, 500 + 10 * k + int(10 * p) + seed)
        for off in (0, 12345):
            want = O.accept_sample(t, dl, drafts, 0.7, 0xC0FFEE + seed, off, 2048)
            out = torch.zeros(3, dtype=torch.int32, device="cuda")
            ctx.accept_sample(dev(t), dev(dl), dev(drafts), 0.7, 0xC0FFEE + seed, off, 2048, out)
            ctx.synchronize()
            assert list(host(out)) == list(want), (seed, off)
