"""GPU parity of the PLE n-gram block (mtpx_ple_*, mtpx_ngram_row_ids) against the
oracle composition (oracle.ple_forward), bit-exact through the C ABI: row ids over
histories with eos tokens and out-of-vocabulary ids, the embedding rows, the block
output and the stream sum over windows with partial commits, a discarded window and
state load/store, at the model's geometry and at a small one."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16  # noqa: E402

EOS = 248044


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def _cfg(mtpx, H, hc, E, hpn, gs, base):
    return mtpx.PLEConfig(hidden=H, hc=hc, embed_dim=E, ngram_size=3, heads_per_ngram=hpn, conv_kernel=4,
                          group_size=gs, row_group_size=32, eos=EOS, vocab_base=base, token_vocab=248320, eps=1e-6)


GEOMS = [
    # the model's geometry (hidden 2560, 4 streams, 16 heads of 160), a small table
    dict(H=2560, hc=4, E=2560, hpn=8, gs=64, base=2000),
    dict(H=2560, hc=4, E=2560, hpn=8, gs=32, base=1000),
    # a small one: hidden 256, 2 streams, 4 heads of 64
    dict(H=256, hc=2, E=256, hpn=2, gs=32, base=300),
]


def _history(r, n, eos_every=5):
    h = r.integers(0, 248320, n).astype(np.int32)
    h[r.integers(0, n, max(1, n // eos_every))] = EOS
    return h


@pytest.mark.parametrize("geom", GEOMS[::2], ids=["model", "small"])
def test_ngram_row_ids_bit_exact(ctx, geom):
    import mtpx
    from oracle.target_ref import download_ple, ple_cfg_dict
    cfg = _cfg(mtpx, **geom)
    ple = mtpx.PLE(ctx, cfg, seed=3)
    w = download_ple(ple.weights(), cfg)
    nh = 2 * geom["hpn"]
    assert w["table"][0].shape[0] == sum(O.primes_above(geom["base"], nh))
    r = np.random.default_rng(7)
    for S in range(1, 9):
        hist = _history(r, 2 + S)
        if S == 3:
            hist[:] = EOS  # a fresh request: the context is eos
        if S == 5:
            hist[4] = -7        # out of the vocabulary: flagged, not read
            hist[5] = 2 ** 31 - 1
        print("case row ids", geom, S, flush=True)
        out = torch.zeros(S, nh, dtype=torch.int32, device="cuda")
        ple.row_ids(dev(hist), S, out)
        want = O.ngram_row_ids(hist, 2, 3, geom["hpn"], w["mult"], w["vocab"], w["offs"], w["table"][0].shape[0],
                               EOS)
        assert np.array_equal(host(out), want)
        assert ((want >= -1) & (want < w["table"][0].shape[0])).all()
    ple.close()


@pytest.mark.parametrize("geom", GEOMS, ids=["model-gs64", "model-gs32", "small"])
def test_ple_forward_windows_bit_exact(ctx, geom):
    import mtpx
    from oracle.target_ref import download_ple, ple_cfg_dict
    cfg = _cfg(mtpx, **geom)
    ple = mtpx.PLE(ctx, cfg, seed=11)
    st = mtpx.PLEState(ctx, cfg)
    w = download_ple(ple.weights(), cfg)
    oc = ple_cfg_dict(cfg)
    W, E, nb = geom["hc"] * geom["H"], geom["E"], 9
    r = np.random.default_rng(geom["H"] + geom["gs"])
    # fresh state: zero conv rows, eos context
    conv, context = np.zeros((nb, W), np.uint16), np.full(2, EOS, np.int32)

    def window(ids, commit):
        S = len(ids)
        stream = rand_bf16(r, (S, W))
        out, tot, emb = empty_bf16(S, W), empty_bf16(S, W), empty_bf16(S, E)
        ple.forward(st, dev(np.asarray(ids, np.int32)), dev(stream), out, tot, emb)
        want = O.ple_forward(w, oc, stream, ids, conv, context)
        assert np.array_equal(host(emb), want["embedded"])
        assert np.array_equal(host(out), want["out"])
        assert np.array_equal(host(tot), want["sum"])
        if commit is not None:
            st.commit(commit)
            return O.ple_advance(want, commit, nb, 2)
        return conv, context

    print("case ple window A (fresh)", geom, flush=True)
    conv, context = window([5, 900, EOS, 33], 2)
    print("case ple window B", flush=True)
    conv, context = window(list(_history(r, 3)), 3)
    print("case ple window C (discarded)", flush=True)
    window(list(_history(r, 8)), None)
    print("case ple window D (after the discard)", flush=True)
    conv, context = window(list(_history(r, 1)), 1)
    # the committed state, materialised, and a reload of it
    c_dev, x_dev = empty_bf16(nb, W), torch.zeros(2, dtype=torch.int32, device="cuda")
    st.store(c_dev, x_dev)
    assert np.array_equal(host(c_dev), conv)
    assert np.array_equal(host(x_dev), context)
    conv = rand_bf16(r, (nb, W))
    context = np.array([17, 248319], np.int32)
    st.load(dev(conv), dev(context))
    print("case ple window E (loaded state)", flush=True)
    conv, context = window(list(_history(r, 6)), 6)
    assert st.info() == (6, 6)
    with pytest.raises(mtpx.MtpxError):
        st.commit(7)
    ple.close()
    st.close()


def test_ple_refuses_bad_geometry(ctx):
    import mtpx
    with pytest.raises(mtpx.MtpxError):
        mtpx.PLE(ctx, _cfg(mtpx, H=2000, hc=4, E=2560, hpn=8, gs=64, base=100), seed=1)  # hidden % 256
    with pytest.raises(mtpx.MtpxError):
        mtpx.PLE(ctx, _cfg(mtpx, H=2560, hc=4, E=2400, hpn=8, gs=64, base=100), seed=1)  # embed_dim % 256
