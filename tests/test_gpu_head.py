"""GPU parity of the MTP head's draft step and of the shortlist argmax against the
oracle, through the C ABI, bit-exact: embedding rows, the two projections, the
three hyper-connection mixers, the attention + MoE layer with its own KV cache,
and the shortlist lm_head argmax, over consecutive draft steps (the second step
feeds the first step's multi stream and draft id back in, as the drafter does)
and a rollback."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, qweights, rand_bf16  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


# ---------------------------------------------------------------------------- a18
@pytest.mark.parametrize("rows,H,gs", [(1000, 256, 32), (98584 // 8, 2560, 32), (4096, 2560, 64)])
def test_shortlist_argmax_bit_exact(ctx, rows, H, gs):
    print("case shortlist", rows, H, gs, flush=True)
    r = np.random.default_rng(rows + H)
    wq, s, b = qweights(r, rows, H, gs)
    x = rand_bf16(r, (1, H))
    ids = np.sort(r.choice(1 << 20, rows, replace=False)).astype(np.int32)
    y, _ = O.qmv(wq, s, b, gs, x)
    want = O.shortlist_argmax(y, ids)
    ds, db = dev(s), dev(b)
    for sb in (None, ctx.pack_sb(ds, db, H, gs)):
        out = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        ctx.shortlist_argmax(dev(x)[0], dev(wq), ds, db, gs, dev(ids), out, sb=sb)
        assert int(host(out)[0]) == want


def test_shortlist_argmax_tie_takes_lowest_position(ctx):
    r = np.random.default_rng(9)
    rows, H, gs = 600, 256, 32
    wq, s, b = qweights(r, rows, H, gs)
    # rows 17 and 450 identical and dominant: equal logits, the lower position wins
    b[17] = O.f32_to_bf16(np.full(H // gs, 0.5, np.float32))
    wq[450], s[450], b[450] = wq[17], s[17], b[17]
    x = O.f32_to_bf16(np.abs(r.standard_normal((1, H))).astype(np.float32))
    ids = np.arange(rows, dtype=np.int32) * 3
    y, _ = O.qmv(wq, s, b, gs, x)
    assert O.shortlist_argmax(y, ids) == ids[17]
    out = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    ctx.shortlist_argmax(dev(x)[0], dev(wq), dev(s), dev(b), gs, dev(ids), out)
    assert int(host(out)[0]) == ids[17]


# ---------------------------------------------------------------------------- a17
@pytest.mark.parametrize("gs", [32, 64])
def test_head_draft_steps_bit_exact(ctx, gs):
    import mtpx
    from oracle.head_ref import download_head, oracle_head
    layer = dict(LAYER, group_size=gs)
    hc, lowrank, vocab = 4, 64, 1000
    hcfg = mtpx.HeadConfig(mtpx.LayerConfig(**layer), hc, lowrank, vocab, 500, 980)
    head = mtpx.MTPHead(ctx, hcfg, seed=11 + gs)
    w = head.weights()
    cfg = dict(layer, hc=hc, lowrank=lowrank, vocab=vocab)
    ow = download_head(w, cfg)
    assert w.shortlist_rows == 520 and ow["shortlist_ids"][499] == 499 and ow["shortlist_ids"][500] == 980
    kv = mtpx.KVCache(ctx, layer["kv_heads"], layer["head_dim"], layer["max_positions"])
    HK, D, P, H = layer["kv_heads"], layer["head_dim"], layer["max_positions"], layer["hidden"]
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    r = np.random.default_rng(gs)
    # round 1: a trusted flush of 3 inputs, then two chained draft steps; rollback; round 2
    ids = r.integers(0, vocab, 3).astype(np.int32)
    multi = rand_bf16(r, (3, hc * H))
    plan = [("step", ids, multi), ("chain",), ("chain",), ("trim", 2), ("step", None, None)]
    pos = 0
    last = None
    for item in plan:
        if item[0] == "trim":
            assert kv.trim(item[1]) == item[1]
            pos -= item[1]
            continue
        if item[0] == "chain":
            ids_s = np.array([last[2]], np.int32)
            multi_s = last[0][-1:]
        elif item[1] is None:
            ids_s = r.integers(0, vocab, 2).astype(np.int32)
            multi_s = rand_bf16(r, (2, hc * H))
        else:
            ids_s, multi_s = item[1], item[2]
        S = len(ids_s)
        print("case head gs", gs, item[0], "S", S, "pos", pos, flush=True)
        want = oracle_head(ow, cfg, kc, vc, ids_s, multi_s, pos)
        mn = empty_bf16(S, hc * H)
        sm = empty_bf16(S, H)
        dr = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        head.forward(kv, dev(ids_s), dev(multi_s), mn, sm, dr)
        ctx.synchronize()
        pos += S
        assert kv.offset == pos
        assert np.array_equal(host(mn), want[0])
        assert np.array_equal(host(sm), want[1])
        assert int(host(dr)[0]) == want[2]
        last = want
    kv.close()
    head.close()


def test_head_rejects_bad_arguments(ctx):
    import mtpx
    hcfg = mtpx.HeadConfig(mtpx.LayerConfig(**LAYER), 4, 48, 1000, 500, 980)  # lowrank % 32 != 0
    with pytest.raises(mtpx.MtpxError):
        mtpx.MTPHead(ctx, hcfg, seed=1)
