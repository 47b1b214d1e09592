"""GPU parity at the shapes the benchmark runs, bit-exact through the C ABI against the
oracle: the MoE block at 512 experts / top-10 / width 640 / hidden 2560, one full decoder
layer (config 3: 24/2 heads x 256 over 1024 cached positions), the MTP head at full
dims with the whole 98,584-row shortlist, and the target's verify forward at full width
(hidden 2560, hyper-connections 4 x 2560 with rank 320, GDN 16/48 heads, the PLE block
with its full 320,001,446-row table, vocab 248,320) -- 48 layers at gs64 (config 4) and
4 layers at gs32 -- over a synthetic committed prefix of 1024 positions, a verify window,
a partial commit and the next window.

The oracle reads weights from the device lazily (routed experts, embedding rows and
n-gram table rows only as it uses them), so the full model is never copied to the host."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16, write_device  # noqa: E402

# fixtures/qwen3_8_125b_a6b_config.json (text_config) of the reference
FULL = dict(hidden=2560, experts=512, top_k=10, expert_width=640, heads=24, kv_heads=2, head_dim=256, rot_dims=64,
            index_dim=128, rope_theta=1e7, eps=1e-6)
LINEAR = dict(key_heads=16, value_heads=48, conv_kernel=4, full_attention_interval=4, hc=4, lowrank=320,
              vocab=248320)
PREFIX = 1024


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def _differ(got, want):
    d = np.abs(O.bf16_to_f32(got).astype(np.float64) - O.bf16_to_f32(want).astype(np.float64))
    return f"{int((got != want).sum())} of {got.size} differ, max |diff| {d.max():.3g}"


# ---------------------------------------------------------------------------- MoE, E = 512
@pytest.mark.parametrize("gs", [64, 32])
def test_moe_full_shape_bit_exact(ctx, gs):
    import mtpx
    from oracle.layer_ref import download_moe
    cfg = dict(FULL, group_size=gs, max_positions=64)
    layer = mtpx.DecoderLayer(ctx, mtpx.LayerConfig(**cfg), seed=0x5EED0003 + gs)
    lw = layer.weights()
    moe = download_moe(lw.moe, cfg, lazy=True)
    H, E, K, F = FULL["hidden"], FULL["experts"], FULL["top_k"], FULL["expert_width"]
    r = np.random.default_rng(gs)
    for M in (1, 2, 4, 6, 8):
        print("case moe full gs", gs, "M", M, flush=True)
        x = rand_bf16(r, (M, H))
        from oracle.layer_ref import moe_y
        moe_y(moe, x, H, E, K, F, gs)  # fetches the routed experts
        want = O.moe_block(moe, x, H, E, K, F, gs)
        y = empty_bf16(M, H)
        idx = torch.full((M, K), -1, dtype=torch.int32, device="cuda")
        wts = torch.zeros(M, K, dtype=torch.float32, device="cuda")
        nu = torch.zeros(1, dtype=torch.int32, device="cuda")
        ctx.moe_forward(lw.moe, dev(x), y, idx, wts, None, nu)
        ctx.synchronize()
        assert np.array_equal(host(idx), want["idx"])
        assert np.array_equal(host(wts), want["w"])
        assert int(host(nu)[0]) == len(np.unique(want["idx"]))
        got = host(y)
        assert np.array_equal(got, want["y"]), _differ(got, want["y"])
    layer.close()


# ---------------------------------------------------------------------------- config 3: one layer
@pytest.mark.parametrize("gs", [64, 32])
def test_layer_config3_bit_exact(ctx, gs):
    import mtpx
    from oracle.layer_ref import download, oracle_layer
    P = PREFIX + 64
    cfg = dict(FULL, group_size=gs, max_positions=P)
    layer = mtpx.DecoderLayer(ctx, mtpx.LayerConfig(**cfg), seed=0x5EED0003)
    kv = mtpx.KVCache(ctx, cfg["kv_heads"], cfg["head_dim"], P)
    w = download(layer.weights(), cfg, lazy=True)
    HK, D, H = cfg["kv_heads"], cfg["head_dim"], cfg["hidden"]
    r = np.random.default_rng(3 + gs)
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
    vc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
    kp, vp, tmax = kv.buffers()
    assert tmax == P
    write_device(kp, kc)
    write_device(vp, vc)
    kv.offset = PREFIX
    pos = PREFIX
    # (past 1024 positions, four or more tokens take the two-token attention workgroups; five leaves the
    # last group's second half idle)
    for kind, n in [("fwd", 1), ("fwd", 2), ("fwd", 4), ("trim", 3), ("fwd", 6), ("fwd", 5)]:
        print("case layer config3 gs", gs, kind, n, "pos", pos, flush=True)
        if kind == "trim":
            assert kv.trim(n) == n
            pos -= n
            continue
        x = rand_bf16(r, (n, H))
        want = oracle_layer(w, cfg, kc, vc, x, pos)
        y = empty_bf16(n, H)
        layer.forward(kv, dev(x), y)
        ctx.synchronize()
        pos += n
        assert kv.offset == pos
        got = host(y)
        assert np.array_equal(got, want), _differ(got, want)
    kv.close()
    layer.close()


# ---------------------------------------------------------------------------- MTP head, full dims
@pytest.mark.parametrize("gs", [64, 32])
def test_head_full_dims_bit_exact(ctx, gs):
    import mtpx
    from oracle.head_ref import download_head, oracle_head
    P = PREFIX + 64
    layer = dict(FULL, group_size=gs, max_positions=P)
    hc, lowrank, vocab = LINEAR["hc"], LINEAR["lowrank"], LINEAR["vocab"]
    head = mtpx.MTPHead(ctx, mtpx.HeadConfig(mtpx.LayerConfig(**layer), hc, lowrank, vocab, 98304, 248044),
                        seed=0x5EED0007 + gs)
    hw = head.weights()
    assert hw.shortlist_rows == 98584
    cfg = dict(layer, hc=hc, lowrank=lowrank, vocab=vocab)
    ow = download_head(hw, cfg, lazy=True)
    assert ow["shortlist_ids"][98307] == 98307 and ow["shortlist_ids"][98308] == 248044
    kv = mtpx.KVCache(ctx, layer["kv_heads"], layer["head_dim"], P)
    HK, D, H = layer["kv_heads"], layer["head_dim"], layer["hidden"]
    r = np.random.default_rng(7 + gs)
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
    vc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
    kp, vp, _ = kv.buffers()
    write_device(kp, kc)
    write_device(vp, vc)
    kv.offset = PREFIX
    pos, last = PREFIX, None
    # a trusted flush of 8 inputs, two chained draft steps, a rollback of 2, a flush of 5
    for item in [("flush", 8), ("chain", 1), ("chain", 1), ("trim", 2), ("flush", 5)]:
        if item[0] == "trim":
            assert kv.trim(item[1]) == item[1]
            pos -= item[1]
            continue
        if item[0] == "chain":
            ids_s, multi_s = np.array([last[2]], np.int32), last[0][-1:]
        else:
            ids_s = r.integers(0, vocab, item[1]).astype(np.int32)
            multi_s = rand_bf16(r, (item[1], hc * H))
        S = len(ids_s)
        print("case head full gs", gs, item[0], "S", S, "pos", pos, flush=True)
        want = oracle_head(ow, cfg, kc, vc, ids_s, multi_s, pos)
        mn, sm = empty_bf16(S, hc * H), empty_bf16(S, H)
        dr = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        head.forward(kv, dev(ids_s), dev(multi_s), mn, sm, dr)
        ctx.synchronize()
        pos += S
        assert kv.offset == pos
        got = host(mn)
        assert np.array_equal(got, want[0]), _differ(got, want[0])
        got = host(sm)
        assert np.array_equal(got, want[1]), _differ(got, want[1])
        assert int(host(dr)[0]) == want[2]
        last = want
    kv.close()
    head.close()


# ---------------------------------------------------------------------------- target verify (config 4)
def _target(ctx, gs, layers, P):
    import mtpx
    lc = dict(FULL, group_size=gs, max_positions=P)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**lc), LINEAR["key_heads"], LINEAR["value_heads"], LINEAR["conv_kernel"],
                           layers, LINEAR["full_attention_interval"], LINEAR["hc"], LINEAR["lowrank"], LINEAR["vocab"])
    # the PLE block on layer index 1: ngram_size 3, 8 heads per n-gram, embed dim 2560, 4 taps,
    # table rows 4-bit gs32, eos 248044, head vocabularies the primes above 20,000,000
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=2560, hc=4, embed_dim=2560, ngram_size=3, heads_per_ngram=8, conv_kernel=4,
                            group_size=gs, row_group_size=32, eos=248044, vocab_base=20_000_000, token_vocab=248320,
                            eps=FULL["eps"])
    t = mtpx.Target(ctx, tc, seed=0x5EED0004)
    cfg = dict(lc, **LINEAR, num_layers=layers, ple_layer=1)
    return t, cfg


@pytest.mark.timeout(900)
@pytest.mark.parametrize("gs,layers,windows", [(64, 48, [(4, 2), (3, 3)]), (32, 4, [(6, 5), (1, 1), (2, 0)])],
                         ids=["gs64-48layers", "gs32-4layers"])
def test_target_verify_full_shape_bit_exact(ctx, gs, layers, windows):
    import mtpx
    from oracle.target_ref import download_target, oracle_commit, oracle_verify
    P = PREFIX + 64
    t, cfg = _target(ctx, gs, layers, P)
    print("case target full: weights ready", gs, layers, flush=True)
    ow = download_target(t, cfg, lazy=True)
    kinds = [L["kind"] for L in ow["layers"]]
    assert kinds.count(1) == layers // 4
    st = mtpx.TargetState(ctx, t)
    H, HK, D, hc, V = cfg["hidden"], cfg["kv_heads"], cfg["head_dim"], cfg["hc"], cfg["vocab"]
    r = np.random.default_rng(100 + layers)
    ostate = dict(kc={}, vc={}, conv={}, ssm={})
    for i, kind in enumerate(kinds):
        if kind == 1:
            kc = np.zeros((HK, P, D), np.uint16)
            vc = np.zeros_like(kc)
            kc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
            vc[:, :PREFIX] = rand_bf16(r, (HK, PREFIX, D))
            kp, vp, _ = st.kv(i).buffers()
            write_device(kp, kc)
            write_device(vp, vc)
            ostate["kc"][i], ostate["vc"][i] = kc, vc
        else:
            g = ow["layers"][i]["gdn"]["geom"]
            conv = rand_bf16(r, (g.kc - 1, g.conv_dim))
            ssm = (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(np.float32)
            st.gdn(i).load(dev(conv), dev(ssm))
            ostate["conv"][i], ostate["ssm"][i] = conv, ssm
    conv = rand_bf16(r, (9, hc * H))
    context = r.integers(0, V, 2).astype(np.int32)
    st.ple().load(dev(conv), dev(context))
    ostate["ple"] = (conv, context)
    st.set_offset(PREFIX)
    torch.cuda.synchronize()
    pos = PREFIX
    for S, keep in windows:
        print("case target full gs", gs, "layers", layers, "window", S, "pos", pos, flush=True)
        ids = r.integers(0, V, S).astype(np.int32)
        lg, mt, mx = empty_bf16(S, V), empty_bf16(S, hc * H), empty_bf16(S, H)
        t.verify(st, dev(ids), lg, mt, mx)
        want = oracle_verify(ow, cfg, ostate, ids, pos)
        got = host(mx)
        assert np.array_equal(got, want[2]), _differ(got, want[2])
        got = host(mt)
        assert np.array_equal(got, want[1]), _differ(got, want[1])
        got = host(lg)
        assert np.array_equal(got, want[0]), _differ(got, want[0])
        st.commit(keep)
        oracle_commit(ow, cfg, ostate, want[3], keep)
        pos += keep
        assert st.info() == (pos, 0)
    st.close()
    t.close()
