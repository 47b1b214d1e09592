"""GPU parity of the target prefill (mtpx_target_prefill), bit-exact through the C ABI: a prompt
batch gives every position's multi stream and the last position's logits exactly as verifying and
committing it in windows of 8 does, and leaves the same state (the next verify is bit-equal).
Against the oracle composition's windows at small dims (a prompt of two full windows and a tail,
with the PLE block), against the GPU's own windowed verify path for a prompt of 600 positions
(two prefill batches, 75 windows, the batched MoE launches) and at full width (hidden 2560, 512
experts, hyper-connections 4 x 2560, the full PLE table, 4 layers): 45 positions over a
1024-position prefix, 600 positions (the benched batch of 512, then 88), and a prompt after a
partly committed verify window; and the MTP head over a batch of backlog positions (the drafter's
flush) against windows of 8."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16, write_device  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=700)
TARGET = dict(key_heads=1, value_heads=2, conv_kernel=4, num_layers=5, full_attention_interval=4, hc=4, lowrank=64,
              vocab=1000)


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def _small_target(ctx, seed):
    import mtpx
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**LAYER), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], embed_dim=256, ngram_size=3, heads_per_ngram=2,
                            conv_kernel=4, group_size=LAYER["group_size"], row_group_size=32, eos=7, vocab_base=300,
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"])
    cfg = dict(LAYER, **TARGET, ple_layer=1)
    return mtpx.Target(ctx, tc, seed=seed), cfg


def _load_prefix(st, kinds, gdn_geoms, cfg, pre, seed):
    """A random committed prefix of `pre` positions (K/V rows, GDN conv rows and state, PLE conv rows and
    context), the same for every state given the same seed; returns it in the oracle's layout."""
    H, HK, D, P, hc, V = cfg["hidden"], cfg["kv_heads"], cfg["head_dim"], cfg["max_positions"], cfg["hc"], cfg["vocab"]
    r = np.random.default_rng(seed)
    ostate = dict(kc={}, vc={}, conv={}, ssm={})
    for i, kind in enumerate(kinds):
        if kind == 1:
            kc = np.zeros((HK, P, D), np.uint16)
            vc = np.zeros_like(kc)
            kc[:, :pre] = rand_bf16(r, (HK, pre, D))
            vc[:, :pre] = rand_bf16(r, (HK, pre, D))
            kp, vp, _ = st.kv(i).buffers()
            write_device(kp, kc)
            write_device(vp, vc)
            ostate["kc"][i], ostate["vc"][i] = kc, vc
        else:
            g = gdn_geoms[i]
            conv = rand_bf16(r, (g.kc - 1, g.conv_dim))
            ssm = (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(np.float32)
            st.gdn(i).load(dev(conv), dev(ssm))
            ostate["conv"][i], ostate["ssm"][i] = conv, ssm
    conv = rand_bf16(r, (9, hc * H))
    context = r.integers(0, V, 2).astype(np.int32)
    st.ple().load(dev(conv), dev(context))
    ostate["ple"] = (conv, context)
    st.set_offset(pre)
    torch.cuda.synchronize()
    return ostate


def _windows(t, st, ids, V, W):
    """The windowed path: verify + commit in windows of 8; every position's multi stream and the last logits."""
    multi = []
    for w0 in range(0, len(ids), 8):
        w = ids[w0:w0 + 8]
        lg, mt = empty_bf16(len(w), V), empty_bf16(len(w), W)
        t.verify(st, dev(w), lg, mt)
        st.commit(len(w))
        multi.append(host(mt))
    return np.concatenate(multi), host(lg)[-1]


def _prefill(t, st, ids, V, W):
    lg, mt = empty_bf16(V), empty_bf16(len(ids), W)
    t.prefill(st, dev(ids), lg, mt)
    return host(mt), host(lg)


def test_prefill_matches_oracle_windows(ctx):
    import mtpx
    from oracle.target_ref import download_target, oracle_commit, oracle_verify
    t, cfg = _small_target(ctx, 31)
    ow = download_target(t, cfg)
    kinds = [L["kind"] for L in ow["layers"]]
    geoms = {i: L["gdn"]["geom"] for i, L in enumerate(ow["layers"]) if L["kind"] == 0}
    V, W = cfg["vocab"], cfg["hc"] * cfg["hidden"]
    st = mtpx.TargetState(ctx, t)
    pre = 9
    ostate = _load_prefix(st, kinds, geoms, cfg, pre, 5)
    r = np.random.default_rng(3)
    ids = r.integers(0, V, 21).astype(np.int32)
    ids[4] = 7  # the PLE block's eos inside the prompt
    print("case prefill 21 vs oracle windows", flush=True)
    got_mt, got_lg = _prefill(t, st, ids, V, W)
    assert st.info() == (pre + 21, 0)
    want_mt = []
    pos = pre
    for w0 in range(0, 21, 8):
        w = ids[w0:w0 + 8]
        want = oracle_verify(ow, cfg, ostate, w, pos)
        oracle_commit(ow, cfg, ostate, want[3], len(w))
        want_mt.append(want[1])
        pos += len(w)
    assert np.array_equal(got_mt, np.concatenate(want_mt))
    assert np.array_equal(got_lg, want[0][-1])
    print("case prefill then verify", flush=True)
    nxt = np.array([11, 7, 500, 2], np.int32)
    lg, mt = empty_bf16(4, V), empty_bf16(4, W)
    t.verify(st, dev(nxt), lg, mt)
    want = oracle_verify(ow, cfg, ostate, nxt, pos)
    assert np.array_equal(host(mt), want[1])
    assert np.array_equal(host(lg), want[0])
    st.close()
    t.close()


def test_prefill_two_batches_matches_windows(ctx):
    """600 positions: two prefill batches (512 + 88), 75 full windows; then a prefill of 3 more positions
    (one short window) and a verify, each against the windowed path's state."""
    import mtpx
    from oracle.target_ref import download_target
    t, cfg = _small_target(ctx, 41)
    ow = download_target(t, cfg)
    kinds = [L["kind"] for L in ow["layers"]]
    geoms = {i: L["gdn"]["geom"] for i, L in enumerate(ow["layers"]) if L["kind"] == 0}
    V, W = cfg["vocab"], cfg["hc"] * cfg["hidden"]
    a, b = mtpx.TargetState(ctx, t), mtpx.TargetState(ctx, t)
    pre = 17
    _load_prefix(a, kinds, geoms, cfg, pre, 8)
    _load_prefix(b, kinds, geoms, cfg, pre, 8)
    r = np.random.default_rng(4)
    for n in (600, 3):
        ids = r.integers(0, V, n).astype(np.int32)
        ids[r.integers(0, n, max(1, n // 50))] = 7
        print("case prefill", n, "vs windows", flush=True)
        got_mt, got_lg = _prefill(t, a, ids, V, W)
        want_mt, want_lg = _windows(t, b, ids, V, W)
        assert np.array_equal(got_mt, want_mt)
        assert np.array_equal(got_lg, want_lg)
        assert a.info() == b.info()
    nxt = dev(np.array([5, 6, 7, 8, 9], np.int32))
    la, lb = empty_bf16(5, V), empty_bf16(5, V)
    t.verify(a, nxt, la)
    t.verify(b, nxt, lb)
    assert np.array_equal(host(la), host(lb))
    print("case prefill refusals", flush=True)
    with pytest.raises(mtpx.MtpxError, match="cache full"):
        t.prefill(a, dev(np.zeros(LAYER["max_positions"], np.int32)))
    with pytest.raises(mtpx.MtpxError):
        t.prefill(a, dev(np.zeros(0, np.int32)))
    a.close()
    b.close()
    t.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("pre,n,partial", [(1024, 45, False), (400, 600, False), (300, 70, True)],
                         ids=["45-after-1024", "600-after-400", "70-after-partial-window"])
def test_prefill_full_width_matches_windows(ctx, pre, n, partial):
    """Full width, 4 layers at gs64 (GDN 16/48 heads, attention 24/2 x 256, 512 experts top-10, the PLE
    block with its full table): a 45-position prompt after a 1024-position prefix; 600 positions (a
    batch of 512 at the benched size, then 88) after 400; and a prompt after a verify window of 5 of
    which 3 positions were committed (the batch GDN kernel replays the committed journal steps and
    reads the conv rows of that window)."""
    import mtpx
    from oracle.target_ref import download_target
    FULL = dict(hidden=2560, experts=512, top_k=10, expert_width=640, heads=24, kv_heads=2, head_dim=256,
                rot_dims=64, index_dim=128, rope_theta=1e7, eps=1e-6, group_size=64, max_positions=1100)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**FULL), 16, 48, 4, 4, 4, 4, 320, 248320)
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=2560, hc=4, embed_dim=2560, ngram_size=3, heads_per_ngram=8, conv_kernel=4,
                            group_size=64, row_group_size=32, eos=248044, vocab_base=20_000_000, token_vocab=248320,
                            eps=FULL["eps"])
    t = mtpx.Target(ctx, tc, seed=0x5EED0009)
    cfg = dict(FULL, key_heads=16, value_heads=48, conv_kernel=4, num_layers=4, full_attention_interval=4, hc=4,
               lowrank=320, vocab=248320, ple_layer=1)
    ow = download_target(t, cfg, lazy=True)
    kinds = [L["kind"] for L in ow["layers"]]
    geoms = {i: L["gdn"]["geom"] for i, L in enumerate(ow["layers"]) if L["kind"] == 0}
    V, W = cfg["vocab"], cfg["hc"] * cfg["hidden"]
    a, b = mtpx.TargetState(ctx, t), mtpx.TargetState(ctx, t)
    _load_prefix(a, kinds, geoms, cfg, pre, 12)
    _load_prefix(b, kinds, geoms, cfg, pre, 12)
    if partial:
        first = dev(np.array([11, 12, 13, 14, 15], np.int32))
        la, lb = empty_bf16(5, V), empty_bf16(5, V)
        t.verify(a, first, la)
        t.verify(b, first, lb)
        a.commit(3)
        b.commit(3)
        assert np.array_equal(host(la), host(lb))
    ids = np.random.default_rng(6 + n).integers(0, V, n).astype(np.int32)
    print("case prefill full width", n, "after", pre, "partial", partial, flush=True)
    got_mt, got_lg = _prefill(t, a, ids, V, W)
    want_mt, want_lg = _windows(t, b, ids, V, W)
    assert np.array_equal(got_mt, want_mt)
    assert np.array_equal(got_lg, want_lg)
    assert a.info() == b.info() == (pre + (3 if partial else 0) + n, 0)
    nxt = dev(np.array([1, 2, 3, 4], np.int32))
    la, lb = empty_bf16(4, V), empty_bf16(4, V)
    t.verify(a, nxt, la)
    t.verify(b, nxt, lb)
    assert np.array_equal(host(la), host(lb))
    a.close()
    b.close()
    t.close()


@pytest.mark.parametrize("n", [37, 256])
def test_head_batch_matches_windows(ctx, n):
    """The MTP head over a batch of backlog positions (the drafter's flush after a prompt) equals the
    same positions in windows of 8: every multi_next and sample row, the last draft, and the next step
    from the caches they leave."""
    import mtpx
    layer = dict(LAYER, max_positions=400)
    hc, lowrank, vocab = 4, 64, 1000
    head = mtpx.MTPHead(ctx, mtpx.HeadConfig(mtpx.LayerConfig(**layer), hc, lowrank, vocab, 500, 980), seed=19)
    H, W = layer["hidden"], hc * layer["hidden"]
    kva = mtpx.KVCache(ctx, layer["kv_heads"], layer["head_dim"], layer["max_positions"])
    kvb = mtpx.KVCache(ctx, layer["kv_heads"], layer["head_dim"], layer["max_positions"])
    r = np.random.default_rng(n)
    ids = dev(r.integers(0, vocab + 20, n).astype(np.int32))  # a few ids outside the vocabulary
    multi = dev(rand_bf16(r, (n, W)))
    print("case head batch", n, flush=True)
    na, sa, da = empty_bf16(n, W), empty_bf16(n, H), torch.full((1,), -1, dtype=torch.int32, device="cuda")
    head.forward(kva, ids, multi, na, sa, da)
    nb, sb = empty_bf16(n, W), empty_bf16(n, H)
    db = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    for w0 in range(0, n, 8):
        w1 = min(n, w0 + 8)
        head.forward(kvb, ids[w0:w1], multi[w0:w1], nb[w0:w1], sb[w0:w1], db if w1 == n else None)
    assert np.array_equal(host(na), host(nb))
    assert np.array_equal(host(sa), host(sb))
    assert int(host(da)[0]) == int(host(db)[0])
    assert kva.offset == kvb.offset == n
    step_ids, step_multi = ids[:1], multi[:1]
    oa, ob = empty_bf16(1, W), empty_bf16(1, W)
    xa, xb = torch.full((1,), -1, dtype=torch.int32, device="cuda"), torch.full((1,), -1, dtype=torch.int32, device="cuda")
    head.forward(kva, step_ids, step_multi, oa, None, xa)
    head.forward(kvb, step_ids, step_multi, ob, None, xb)
    assert np.array_equal(host(oa), host(ob)) and int(host(xa)[0]) == int(host(xb)[0])
    with pytest.raises(mtpx.MtpxError):
        head.forward(kva, dev(np.zeros(257, np.int32)), dev(np.zeros((257, W), np.uint16)), empty_bf16(257, W))
    kva.close()
    kvb.close()
    head.close()
