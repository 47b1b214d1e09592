"""GPU parity of the gated-deltanet sublayer (mtpx_gdn_*) against the oracle,
bit-exact through the C ABI: the core (prep, recurrence, gated RMS) at the
model's GDN dims from a loaded random state; windows with partial commits and
discarded windows against one sequential oracle pass over the committed
positions; the whole sublayer (in_proj GEMV, core, out_proj GEMV); refused
calls."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, read_device  # noqa: E402

QWEN = dict(hidden=2560, key_heads=16, value_heads=48, conv_kernel=4, group_size=64, eps=1e-6)
SMALL = dict(hidden=1024, key_heads=4, value_heads=12, conv_kernel=4, group_size=32, eps=1e-6)


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def download(w, cfg, g):
    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(q4, rows, K):
        gs = cfg["group_size"]
        return (read_device(q4.w, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(q4.s, rows * K // gs).reshape(rows, K // gs), bf(q4.b, rows * K // gs).reshape(rows, K // gs))

    hv = cfg["value_heads"]
    return dict(in_proj=q(w.in_proj, g.proj_w, cfg["hidden"]), out_proj=q(w.out_proj, cfg["hidden"], hv * 128),
                conv_w=bf(w.conv_w, g.conv_dim * g.kc).reshape(g.conv_dim, g.kc),
                nea=read_device(w.neg_exp_alog, 4 * hv, np.float32), dtb=bf(w.dt_bias, hv), nw=bf(w.norm_w, 128))


def setup(ctx, cfg, seed):
    import mtpx
    gc = mtpx.GDNConfig(**cfg)
    layer = mtpx.GDN(ctx, gc, seed)
    st = mtpx.GDNState(ctx, gc)
    g = O.gdn_geom(cfg["key_heads"], cfg["value_heads"], cfg["conv_kernel"])
    return layer, st, g, download(layer.weights(), cfg, g)


def rand_state(r, g):
    conv = O.f32_to_bf16(r.standard_normal((g.kc - 1, g.conv_dim)).astype(np.float32))
    ssm = (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(np.float32)
    return conv, ssm


def oracle_core(g, ow, proj, conv, ssm, eps):
    return O.gdn_core(g, proj, conv, ssm, ow["conv_w"], ow["nea"], ow["dtb"], ow["nw"], eps)


def stored(st, g):
    conv = empty_bf16(g.kc - 1, g.conv_dim)
    ssm = torch.zeros(g.hv, 128, 128, dtype=torch.float32, device="cuda")
    st.store(conv, ssm)
    return host(conv), host(ssm)


# ---------------------------------------------------------------------------- core
@pytest.mark.parametrize("S", [1, 4, 8])
def test_gdn_core_bit_exact(ctx, S):
    print("case gdn core S", S, flush=True)
    layer, st, g, ow = setup(ctx, QWEN, 21)
    r = np.random.default_rng(S)
    conv, ssm = rand_state(r, g)
    st.load(dev(conv), dev(ssm))
    proj = O.f32_to_bf16(r.standard_normal((S, g.proj_w)).astype(np.float32))
    gated = empty_bf16(S, g.hv * 128)
    layer.core(st, dev(proj), gated)
    want = oracle_core(g, ow, proj, conv, ssm, QWEN["eps"])
    assert np.array_equal(host(gated), want["gated"])
    # nothing committed yet: the stored state is the loaded one
    c0, s0 = stored(st, g)
    assert np.array_equal(c0, conv) and np.array_equal(s0, ssm)
    st.commit(S)
    c1, s1 = stored(st, g)
    assert np.array_equal(c1, want["conv_state"])
    assert np.array_equal(s1, want["ssm"])
    st.close()
    layer.close()


def test_gdn_windows_commit_and_discard(ctx):
    layer, st, g, ow = setup(ctx, SMALL, 5)
    r = np.random.default_rng(7)
    conv, ssm = rand_state(r, g)
    st.load(dev(conv), dev(ssm))
    P = lambda n: O.f32_to_bf16(r.standard_normal((n, g.proj_w)).astype(np.float32))  # noqa: E731
    A, B, Cw, D = P(4), P(3), P(2), P(1)
    eps = SMALL["eps"]

    def core(proj):
        out = empty_bf16(proj.shape[0], g.hv * 128)
        layer.core(st, dev(proj), out)
        return host(out)

    print("case gdn windows", flush=True)
    core(A)
    st.commit(2)
    assert st.info() == (4, 2)
    got_b = core(B)
    ref_a2 = oracle_core(g, ow, A[:2], conv, ssm, eps)
    ref_b = oracle_core(g, ow, B, ref_a2["conv_state"], ref_a2["ssm"], eps)
    assert np.array_equal(got_b, ref_b["gated"])
    assert st.info() == (3, 0)
    st.commit(3)
    c, s = stored(st, g)
    assert np.array_equal(c, ref_b["conv_state"]) and np.array_equal(s, ref_b["ssm"])
    # a window with nothing committed is discarded by the next one
    core(Cw)
    got_d = core(D)
    ref_d = oracle_core(g, ow, D, ref_b["conv_state"], ref_b["ssm"], eps)
    assert np.array_equal(got_d, ref_d["gated"])
    st.commit(1)
    c, s = stored(st, g)
    assert np.array_equal(c, ref_d["conv_state"]) and np.array_equal(s, ref_d["ssm"])
    st.close()
    layer.close()


# ---------------------------------------------------------------------------- whole sublayer
@pytest.mark.parametrize("cfg,S", [(QWEN, 4), (SMALL, 1), (SMALL, 6)])
def test_gdn_forward_bit_exact(ctx, cfg, S):
    print("case gdn forward", cfg["hidden"], S, flush=True)
    layer, st, g, ow = setup(ctx, cfg, 31 + S)
    r = np.random.default_rng(100 + S)
    conv, ssm = rand_state(r, g)
    st.load(dev(conv), dev(ssm))
    x = O.f32_to_bf16(r.standard_normal((S, cfg["hidden"])).astype(np.float32))
    y = empty_bf16(S, cfg["hidden"])
    gated = empty_bf16(S, g.hv * 128)
    layer.forward(st, dev(x), y, gated)
    gs = cfg["group_size"]
    proj, _ = O.qmv(*ow["in_proj"], gs, x)
    want = oracle_core(g, ow, proj, conv, ssm, cfg["eps"])
    assert np.array_equal(host(gated), want["gated"])
    y_ref, _ = O.qmv(*ow["out_proj"], gs, want["gated"])
    assert np.array_equal(host(y), y_ref)
    st.close()
    layer.close()


def test_gdn_refuses_bad_calls(ctx):
    import mtpx
    layer, st, g, _ = setup(ctx, SMALL, 1)
    with pytest.raises(mtpx.MtpxError):
        st.commit(1)  # no window yet
    other = mtpx.GDNState(ctx, mtpx.GDNConfig(**dict(SMALL, value_heads=8)))
    with pytest.raises(mtpx.MtpxError):
        layer.core(other, dev(np.zeros((1, g.proj_w), np.uint16)), empty_bf16(1, g.hv * 128))
    with pytest.raises(mtpx.MtpxError):
        mtpx.GDN(ctx, mtpx.GDNConfig(**dict(SMALL, value_heads=10)), 1)  # not a multiple of key_heads
    other.close()
    st.close()
    layer.close()
