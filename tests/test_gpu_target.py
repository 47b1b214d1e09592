"""GPU parity of the target's verify forward (mtpx_target_*) against the oracle
composition, bit-exact through the C ABI: logits, the multi stream and the mixed
row over a layer stack of GDN and attention layers (each with hyper-connection
mixers and MoE), with and without the PLE n-gram block on layer 1, from a random
committed prefix (attention K/V rows, GDN states, PLE conv rows and context),
then a partial commit, a window that is discarded by the next verify, and
refused calls."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16, write_device  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)
TARGET = dict(key_heads=1, value_heads=2, conv_kernel=4, num_layers=5, full_attention_interval=4, hc=4, lowrank=64,
              vocab=1000)


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("ple_layer", [1, -1], ids=["ple", "no-ple"])
def test_target_verify_commit_discard_bit_exact(ctx, ple_layer):
    import mtpx
    from oracle.target_ref import download_target, oracle_commit, oracle_verify
    cfg = dict(LAYER, **TARGET, ple_layer=ple_layer)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**LAYER), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = ple_layer
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], embed_dim=256, ngram_size=3, heads_per_ngram=2,
                            conv_kernel=4, group_size=LAYER["group_size"], row_group_size=32, eos=7, vocab_base=300,
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"])
    t = mtpx.Target(ctx, tc, seed=17)
    ow = download_target(t, cfg)
    kinds = [L["kind"] for L in ow["layers"]]
    assert kinds == [0, 0, 0, 1, 0]
    st = mtpx.TargetState(ctx, t)
    H, HK, D, P, hc, V = LAYER["hidden"], LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"], 4, 1000
    r = np.random.default_rng(11)
    pre = 10
    ostate = dict(kc={}, vc={}, conv={}, ssm={})
    for i, kind in enumerate(kinds):
        if kind == 1:
            kc = np.zeros((HK, P, D), np.uint16)
            vc = np.zeros_like(kc)
            kc[:, :pre] = rand_bf16(r, (HK, pre, D))
            vc[:, :pre] = rand_bf16(r, (HK, pre, D))
            kv = st.kv(i)
            kp, vp, tmax = kv.buffers()
            assert tmax == P
            write_device(kp, kc)
            write_device(vp, vc)
            ostate["kc"][i], ostate["vc"][i] = kc, vc
        else:
            g = ow["layers"][i]["gdn"]["geom"]
            conv = rand_bf16(r, (g.kc - 1, g.conv_dim))
            ssm = (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(np.float32)
            st.gdn(i).load(dev(conv), dev(ssm))
            ostate["conv"][i], ostate["ssm"][i] = conv, ssm
    if ple_layer >= 0:
        conv = rand_bf16(r, (9, hc * H))
        context = np.array([3, 7], np.int32)  # 7 is the eos of this config
        st.ple().load(dev(conv), dev(context))
        ostate["ple"] = (conv, context)
    else:
        with pytest.raises(mtpx.MtpxError):
            st.ple()
    st.set_offset(pre)
    torch.cuda.synchronize()

    def run(ids, pos0):
        S = len(ids)
        lg, mt, mx = empty_bf16(S, V), empty_bf16(S, hc * H), empty_bf16(S, H)
        t.verify(st, dev(np.asarray(ids, np.int32)), lg, mt, mx)
        want = oracle_verify(ow, cfg, ostate, np.asarray(ids, np.int32), pos0)
        assert np.array_equal(host(mt), want[1])
        assert np.array_equal(host(mx), want[2])
        assert np.array_equal(host(lg), want[0])
        return want[3]

    print("case target window A", flush=True)
    win = run([5, 77, 7, 0], pre)
    assert st.info() == (pre, 4)
    st.commit(2)
    oracle_commit(ow, cfg, ostate, win, 2)
    assert st.info() == (pre + 2, 0)
    print("case target window B", flush=True)
    run([123, 456, 789], pre + 2)
    # no commit: the next verify discards window B
    print("case target window C", flush=True)
    win = run([42], pre + 2)
    st.commit(1)
    oracle_commit(ow, cfg, ostate, win, 1)
    assert st.info() == (pre + 3, 0)
    st.commit(0)  # nothing open: no change
    assert st.info() == (pre + 3, 0)
    print("case target window D", flush=True)
    run([1, 2, 3, 4, 5, 6, 7, 8], pre + 3)
    with pytest.raises(mtpx.MtpxError):
        st.commit(9)
    with pytest.raises(mtpx.MtpxError):
        st.kv(0)  # a GDN layer has no KV cache
    with pytest.raises(mtpx.MtpxError):
        st.gdn(3)  # an attention layer has no GDN state
    st.close()
    t.close()


def test_target_refusals_and_reset(ctx):
    """A verify refused before any launch leaves the open window intact (commit still works); a window
    past the indexer budget (2048 positions) is refused; reset returns every cache to the fresh state
    (a verify after reset gives the bits of a verify on a new state)."""
    import mtpx
    layer = dict(LAYER, max_positions=2100)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**layer), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], embed_dim=256, ngram_size=3, heads_per_ngram=2,
                            conv_kernel=4, group_size=LAYER["group_size"], row_group_size=32, eos=7, vocab_base=300,
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"])
    t = mtpx.Target(ctx, tc, seed=23)
    H, hc, V = LAYER["hidden"], TARGET["hc"], TARGET["vocab"]
    ids = dev(np.array([3, 1, 4, 1], np.int32))
    fresh = mtpx.TargetState(ctx, t)
    lg0 = empty_bf16(4, V)
    t.verify(fresh, ids, lg0)
    st = mtpx.TargetState(ctx, t)
    for n in (4, 2):  # advance the state: GDN and PLE states, caches and offset all move
        t.verify(st, ids[:n], empty_bf16(n, V))
        st.commit(n)
    print("case target refusals", flush=True)
    t.verify(st, ids[:3], empty_bf16(3, V))
    with pytest.raises(mtpx.MtpxError):
        t.verify(st, dev(np.zeros(9, np.int32)), empty_bf16(9, V))  # S > 8: refused, nothing launched
    st.commit(2)
    assert st.info() == (8, 0)
    st.set_offset(2046)
    with pytest.raises(mtpx.MtpxError, match="indexer budget"):
        t.verify(st, ids, empty_bf16(4, V))
    t.verify(st, ids[:2], empty_bf16(2, V))  # 2046 + 2 == 2048: served
    print("case target reset", flush=True)
    st.reset()
    assert st.info() == (0, 0)
    lg1 = empty_bf16(4, V)
    t.verify(st, ids, lg1)
    assert np.array_equal(host(lg1), host(lg0))
    st.close()
    fresh.close()
    t.close()
