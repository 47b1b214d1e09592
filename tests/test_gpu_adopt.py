"""GPU tests of weight adoption (mtpx_target_adopt, mtpx_head_adopt): a target and a head built over
caller-owned device tensors (here: the tensors of a random-init target and head, handed over as
pointers, as a checkpoint loader would hand over its loaded arrays) give the same bits as the
originals -- with the caller's packed scale/bias rows, with none (the kernels then read the
checkpoint's bf16 scales and biases), and with rows the library packs itself; missing tensors
and a layer schedule that differs from the config are refused."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from gpu_util import dev, host, need_gpu, rand_bf16  # noqa: E402

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


def _cfg():
    import mtpx
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**LAYER), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], embed_dim=256, ngram_size=3, heads_per_ngram=2,
                            conv_kernel=4, group_size=LAYER["group_size"], row_group_size=32, eos=7, vocab_base=300,
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"])
    return tc


def _strip_sb(obj):
    """Null every packed scale/bias pointer of a weights struct (recursively)."""
    for name, typ in obj._fields_:
        v = getattr(obj, name)
        if isinstance(v, C.Structure):
            _strip_sb(v)
        elif name == "sb" or name.endswith("_sb"):
            setattr(obj, name, None)


def _verify_bits(ctx, t, ids_list):
    import mtpx
    st = mtpx.TargetState(ctx, t)
    out = []
    V, W = TARGET["vocab"], TARGET["hc"] * LAYER["hidden"]
    for ids in ids_list:
        lg = torch.zeros(len(ids), V, dtype=torch.bfloat16, device="cuda")
        mt = torch.zeros(len(ids), W, dtype=torch.bfloat16, device="cuda")
        t.verify(st, dev(np.asarray(ids, np.int32)), lg, mt)
        st.commit(len(ids))
        out += [host(lg), host(mt)]
    st.close()
    return out


@pytest.mark.parametrize("mode", ["caller-sb", "no-sb", "library-sb"])
def test_target_adopt_matches_original(ctx, mode):
    import mtpx
    cfg = _cfg()
    t = mtpx.Target(ctx, cfg, seed=41)
    w = t.weights()
    layers = [t.layer_weights(i) for i in range(TARGET["num_layers"])]
    if mode != "caller-sb":
        _strip_sb(w)
        for L in layers:
            _strip_sb(L)
    a = mtpx.Target.adopt(ctx, cfg, w, layers, pack_sb=(mode == "library-sb"))
    windows = [[5, 77, 7, 0], [123, 9], [42]]
    print("case adopt target", mode, flush=True)
    for x, y in zip(_verify_bits(ctx, t, windows), _verify_bits(ctx, a, windows)):
        assert np.array_equal(x, y)
    a.close()
    t.close()


def test_target_adopt_refusals(ctx):
    import mtpx
    cfg = _cfg()
    t = mtpx.Target(ctx, cfg, seed=43)
    w = t.weights()
    layers = [t.layer_weights(i) for i in range(TARGET["num_layers"])]
    bad = [t.layer_weights(i) for i in range(TARGET["num_layers"])]
    bad[0].gdn.in_proj.w = None
    with pytest.raises(mtpx.MtpxError, match="missing"):
        mtpx.Target.adopt(ctx, cfg, w, bad)
    swapped = list(layers)
    swapped[0], swapped[3] = swapped[3], swapped[0]  # an attention layer where the schedule has GDN
    with pytest.raises(mtpx.MtpxError, match="kind"):
        mtpx.Target.adopt(ctx, cfg, w, swapped)
    w2 = t.weights()
    w2.lm_head.s = None
    with pytest.raises(mtpx.MtpxError, match="missing"):
        mtpx.Target.adopt(ctx, cfg, w2, layers)
    t.close()


@pytest.mark.parametrize("pack_sb", [False, True])
def test_head_adopt_matches_original(ctx, pack_sb):
    import mtpx
    hcfg = mtpx.HeadConfig(mtpx.LayerConfig(**LAYER), TARGET["hc"], TARGET["lowrank"], TARGET["vocab"], 500, 980)
    head = mtpx.MTPHead(ctx, hcfg, seed=45)
    w = head.weights()
    if pack_sb:
        _strip_sb(w)  # the library packs its own rows
    a = mtpx.MTPHead.adopt(ctx, hcfg, w, pack_sb=pack_sb)
    H, hc = LAYER["hidden"], TARGET["hc"]
    r = np.random.default_rng(46)
    ids = dev(r.integers(0, TARGET["vocab"], 3).astype(np.int32))
    multi = dev(rand_bf16(r, (3, hc * H)))
    res = []
    for hd in (head, a):
        kv = mtpx.KVCache(ctx, LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"])
        mn = torch.zeros(3, hc * H, dtype=torch.bfloat16, device="cuda")
        sm = torch.zeros(3, H, dtype=torch.bfloat16, device="cuda")
        dr = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        hd.forward(kv, ids, multi, mn, sm, dr)
        res.append((host(mn), host(sm), int(host(dr)[0])))
        kv.close()
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1]) and res[0][2] == res[1][2]
    a.close()
    head.close()
