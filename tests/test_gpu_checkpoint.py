"""GPU tests of the checkpoint loader (mtpx_target_load / mtpx_head_load) through the C ABI.

A small random checkpoint is written with the tensor names, dtypes and shapes of the family's
inventory (Sources/MLXFastTransform/Qwen4ExpCheckpointValidation.swift:312-510: affine-4-bit U32 +
BF16 scales/biases, BF16 norms and router, I64 n-gram buffers, the q4 shared-expert gate, the embedded
`mtp.*` head, the n-gram table in shards), split over three files.  The loaded target and head are
compared bit for bit with a target and head adopted (mtpx_target_adopt / mtpx_head_adopt) from the same
tensors transformed here in numpy, independently of the loader (norm scale x 1/hc in bf16, GDN
in-projection rows qkv|z|b|a, -exp(A_log), q_proj rows regrouped, the indexer's key rows, the shortlist
rows of lm_head); the loaded target's verify is also checked against the oracle (the q4 shared gate
through the whole stack).  A missing tensor, a wrong shape and n-gram head sizes that differ from the
config are refused."""
import ctypes as C
import json
import struct

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, host, need_gpu, rand_bf16  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)
TARGET = dict(key_heads=1, value_heads=2, conv_kernel=4, num_layers=5, full_attention_interval=4, hc=4, lowrank=64,
              vocab=1000)
PLE = dict(embed_dim=256, ngram_size=3, heads_per_ngram=2, conv_kernel=4, row_group_size=32, eos=7, vocab_base=300)
IDX_HEADS = 2  # indexer query heads of the checkpoint (the key head's rows are the last index_dim)


def _cfgs():
    import mtpx
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**LAYER), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], group_size=LAYER["group_size"],
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"], **PLE)
    hc = mtpx.HeadConfig(mtpx.LayerConfig(**LAYER), TARGET["hc"], TARGET["lowrank"], TARGET["vocab"], 500, 980)
    return tc, hc


# ------------------------------------------------------------------------------------------ the checkpoint
def _make_checkpoint(seed, ngram_vocab, ngram_offsets):
    """name -> numpy array (uint32: U32, uint16: BF16 bit patterns, int64: I64)."""
    r = np.random.default_rng(seed)
    H, gs, E, F = LAYER["hidden"], LAYER["group_size"], LAYER["experts"], LAYER["expert_width"]
    HQ, HK, D, ID = LAYER["heads"], LAYER["kv_heads"], LAYER["head_dim"], LAYER["index_dim"]
    hcn, LW, V = TARGET["hc"], TARGET["lowrank"], TARGET["vocab"]
    W = hcn * H
    hk, hv, kc = TARGET["key_heads"], TARGET["value_heads"], TARGET["conv_kernel"]
    cd, vd = (2 * hk + hv) * 128, hv * 128
    ck = {}

    def q4(stem, lead, K, sigma=0.05, g=gs):
        w, s, b = O.affine_quantize(rand_bf16(r, (int(np.prod(lead)), K), sigma), g)
        ck[stem + ".weight"] = w.reshape(*lead, K // 8)
        ck[stem + ".scales"] = s.reshape(*lead, K // g)
        ck[stem + ".biases"] = b.reshape(*lead, K // g)

    def norm(name, n):
        ck[name] = O.f32_to_bf16((1.0 + 0.2 * r.standard_normal(n)).astype(np.float32))

    def hyper(stem, inject):
        norm(stem + ".hc_norm.weight", W)
        q4(stem + ".input_mix_weight_down", (LW,), W)
        q4(stem + ".input_mix_weight_up", (W,), LW)
        if inject:
            q4(stem + ".block_inject_weight", (hcn,), W)

    def decoder(p, attention):
        hyper(p + "attn_hyper_connection", True)
        hyper(p + "mlp_hyper_connection", True)
        ck[p + "mlp.gate.weight"] = rand_bf16(r, (E, H), 0.05)
        for n in ("gate_proj", "up_proj"):
            q4(p + "mlp.shared_expert." + n, (F,), H)
            q4(p + "mlp.switch_mlp." + n, (E, F), H)
        q4(p + "mlp.shared_expert.down_proj", (H,), F)
        q4(p + "mlp.switch_mlp.down_proj", (E, H), F)
        q4(p + "mlp.shared_expert_gate", (1,), H, 0.3)
        if attention:
            norm(p + "self_attn.q_norm.weight", D)
            norm(p + "self_attn.k_norm.weight", D)
            q4(p + "self_attn.q_proj", (2 * HQ * D,), H)
            q4(p + "self_attn.k_proj", (HK * D,), H)
            q4(p + "self_attn.v_proj", (HK * D,), H)
            q4(p + "self_attn.o_proj", (H,), HQ * D)
            q4(p + "self_attn.indexer.index_qk_proj", ((IDX_HEADS + 1) * ID,), H)
            norm(p + "self_attn.indexer.q_layernorm.weight", ID)
            norm(p + "self_attn.indexer.k_layernorm.weight", ID)
        else:
            ck[p + "linear_attn.A_log"] = O.f32_to_bf16((r.standard_normal(hv) * 0.5).astype(np.float32))
            ck[p + "linear_attn.dt_bias"] = rand_bf16(r, (hv,), 0.5)
            ck[p + "linear_attn.conv1d.weight"] = rand_bf16(r, (cd, kc, 1), 0.3)
            norm(p + "linear_attn.norm.weight", 128)
            q4(p + "linear_attn.in_proj_qkv", (cd,), H)
            q4(p + "linear_attn.in_proj_z", (vd,), H)
            q4(p + "linear_attn.in_proj_b", (hv,), H)
            q4(p + "linear_attn.in_proj_a", (hv,), H)
            q4(p + "linear_attn.out_proj", (H,), vd)

    t = "language_model."
    q4(t + "model.embed_tokens", (V,), H, 0.5)
    q4(t + "lm_head", (V,), H)
    hyper(t + "model.hyper_connection_mixer", False)
    for i in range(TARGET["num_layers"]):
        decoder(f"{t}model.layers.{i}.", (i + 1) % TARGET["full_attention_interval"] == 0)
    # the PLE block of layer 1 with its table in three shards
    p = t + "model.layers.1.ple."
    Ed = PLE["embed_dim"]
    nh = (PLE["ngram_size"] - 1) * PLE["heads_per_ngram"]
    rd = Ed // nh
    ck[p + "conv1d.weight"] = rand_bf16(r, (W, PLE["conv_kernel"], 1), 0.3)
    for n in ("norm_conv", "norm_key", "norm_query"):
        norm(p + n + ".weight", W)
    q4(p + "key_proj", (W,), Ed)
    q4(p + "value_proj", (H,), Ed)
    mult = (r.integers(1, 2 ** 40, PLE["ngram_size"]) * 2 + 1).astype(np.int64)
    ck[p + "ple_embedding.layer_multipliers"] = mult
    ck[p + "ple_embedding.ngram_heads_vocab_sizes"] = np.asarray(ngram_vocab, np.int64)
    ck[p + "ple_embedding.ngram_heads_offsets"] = np.asarray(ngram_offsets, np.int64)
    rows = int(np.sum(ngram_vocab)) + 12
    cuts = [0, rows // 3, 2 * rows // 3, rows]
    tw, ts, tb = O.affine_quantize(rand_bf16(r, (rows, rd), 0.5), PLE["row_group_size"])
    for j in range(3):
        s = f"{p}ple_embedding.ngram_embedding.shard_{j}"
        ck[s + ".weight"], ck[s + ".scales"], ck[s + ".biases"] = (tw[cuts[j]:cuts[j + 1]], ts[cuts[j]:cuts[j + 1]],
                                                                   tb[cuts[j]:cuts[j + 1]])
    # the embedded MTP head
    m = t + "mtp."
    norm(m + "pre_fc_norm_embedding.weight", H)
    norm(m + "pre_fc_norm_hidden.weight", W)
    q4(m + "fc_embedding", (H,), H)
    q4(m + "fc_hidden", (H,), H)
    hyper(m + "hyper_connection_mixer", False)
    decoder(m + "layers.0.", True)
    return ck


def _write_safetensors(path, arrays):
    kinds = {np.dtype(np.uint32): "U32", np.dtype(np.uint16): "BF16", np.dtype(np.int64): "I64"}
    hdr, off, blobs = {}, 0, []
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        data = a.tobytes()
        hdr[name] = {"dtype": kinds[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
        blobs.append(data)
    h = json.dumps(hdr, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _write_checkpoint(tmp_path, ck, drop=None, reshape=None):
    names = sorted(n for n in ck if n != drop)
    arrays = {n: (ck[n] if n != reshape else ck[n][:-1]) for n in names}
    files = []
    for j in range(3):
        part = {n: arrays[n] for n in names[j::3]}
        f = tmp_path / f"model-{j + 1:05d}-of-00003.safetensors"
        _write_safetensors(f, part)
        files.append(str(f))
    return files


# ------------------------------------------------------------------------------- the same tensors adopted
class _Dev:
    """Device copies kept alive for the adopted target and head."""

    def __init__(self):
        self.keep = []

    def put(self, a):
        t = dev(np.ascontiguousarray(a))
        self.keep.append(t)
        return t.data_ptr()

    def q4(self, ck, stem, rows=None, order=None):
        import mtpx
        parts = [ck[stem + ".weight"], ck[stem + ".scales"], ck[stem + ".biases"]]
        parts = [p.reshape(-1, p.shape[-1]) for p in parts]
        if order is not None:
            parts = [p[order] for p in parts]
        if rows is not None:
            parts = [p[rows] for p in parts]
        return mtpx.Q4(self.put(parts[0]), self.put(parts[1]), self.put(parts[2]), None)

    def q4_cat(self, ck, stems_rows):
        import mtpx
        cat = [np.concatenate([ck[s + k].reshape(-1, ck[s + k].shape[-1])[rw] for s, rw in stems_rows])
               for k in (".weight", ".scales", ".biases")]
        return mtpx.Q4(self.put(cat[0]), self.put(cat[1]), self.put(cat[2]), None)

    def norm_scale(self, ck, stem):
        x = O.bf16_to_f32(ck[stem + ".hc_norm.weight"])
        return self.put(O.f32_to_bf16(x * np.float32(O.bf16_to_f32(O.f32_to_bf16(np.float32(1.0 / TARGET["hc"]))))))

    def hc(self, ck, stem, inject):
        import mtpx
        h = mtpx.HCWeights()
        h.norm_scale = self.norm_scale(ck, stem)
        h.down = self.q4(ck, stem + ".input_mix_weight_down")
        h.up = self.q4(ck, stem + ".input_mix_weight_up")
        if inject:
            h.inject = self.q4(ck, stem + ".block_inject_weight")
        return h

    def moe(self, ck, p):
        import mtpx
        H, E, K, F, gs = (LAYER[k] for k in ("hidden", "experts", "top_k", "expert_width", "group_size"))
        m = mtpx.MoEWeights(H, E, K, F, gs)
        m.router = self.put(ck[p + "mlp.gate.weight"])
        for ours, theirs in (("gate", "switch_mlp.gate_proj"), ("up", "switch_mlp.up_proj"),
                             ("down", "switch_mlp.down_proj"), ("sh_gate", "shared_expert.gate_proj"),
                             ("sh_up", "shared_expert.up_proj"), ("sh_down", "shared_expert.down_proj"),
                             ("shared_gate", "shared_expert_gate")):
            q = self.q4(ck, p + "mlp." + theirs)
            setattr(m, ours + "_w", q.w)
            setattr(m, ours + "_s", q.s)
            setattr(m, ours + "_b", q.b)
        return m

    def attention(self, ck, p):
        import mtpx
        HQ, HK, D, ID = LAYER["heads"], LAYER["kv_heads"], LAYER["head_dim"], LAYER["index_dim"]
        w = mtpx.LayerWeights()
        order = [h * 2 * D + i for h in range(HQ) for i in range(D)] + [h * 2 * D + D + i for h in range(HQ)
                                                                         for i in range(D)]
        irows = (IDX_HEADS + 1) * ID
        q = self.q4_cat(ck, [(p + "self_attn.q_proj", order), (p + "self_attn.k_proj", slice(None)),
                             (p + "self_attn.v_proj", slice(None)),
                             (p + "self_attn.indexer.index_qk_proj", slice(irows - ID, irows))])
        w.qkv_w, w.qkv_s, w.qkv_b = q.w, q.s, q.b
        w.qkv_rows = 2 * HQ * D + 2 * HK * D + ID
        w.q_norm = self.put(ck[p + "self_attn.q_norm.weight"])
        w.k_norm = self.put(ck[p + "self_attn.k_norm.weight"])
        o = self.q4(ck, p + "self_attn.o_proj")
        w.o_w, w.o_s, w.o_b = o.w, o.s, o.b
        w.moe = self.moe(ck, p)
        return w

    def gdn(self, ck, p):
        import mtpx
        g = mtpx.GDNWeights()
        g.in_proj = self.q4_cat(ck, [(p + "linear_attn.in_proj_" + n, slice(None)) for n in ("qkv", "z", "b", "a")])
        g.conv_w = self.put(ck[p + "linear_attn.conv1d.weight"])
        a_log = O.bf16_to_f32(ck[p + "linear_attn.A_log"]).astype(np.float64)
        g.neg_exp_alog = self.put((-np.exp(a_log)).astype(np.float32))  # exp in double, rounded once
        g.dt_bias = self.put(ck[p + "linear_attn.dt_bias"])
        g.norm_w = self.put(ck[p + "linear_attn.norm.weight"])
        g.out_proj = self.q4(ck, p + "linear_attn.out_proj")
        return g

    def ple(self, ck, p):
        import mtpx
        w = mtpx.PLEWeights()
        w.key_proj = self.q4(ck, p + "key_proj")
        w.value_proj = self.q4(ck, p + "value_proj")
        for n in ("norm_key", "norm_query", "norm_conv"):
            setattr(w, n, self.put(ck[p + n + ".weight"]))
        w.conv_w = self.put(ck[p + "conv1d.weight"])
        shards = [f"{p}ple_embedding.ngram_embedding.shard_{j}" for j in range(3)]
        t = self.q4_cat(ck, [(s, slice(None)) for s in shards])
        w.table.w, w.table.s, w.table.b = t.w, t.s, t.b
        w.table.rows = sum(ck[s + ".weight"].shape[0] for s in shards)
        for k, v in enumerate(ck[p + "ple_embedding.layer_multipliers"]):
            w.table.multiplier[k] = int(v)
        return w


def _adopt(ctx, tc, hcfg, ck):
    import mtpx
    d = _Dev()
    t = "language_model."
    tw = mtpx.TargetWeights()
    tw.embed = d.q4(ck, t + "model.embed_tokens")
    tw.lm_head = d.q4(ck, t + "lm_head")
    tw.final_hc = d.hc(ck, t + "model.hyper_connection_mixer", False)
    layers = []
    for i in range(TARGET["num_layers"]):
        p = f"{t}model.layers.{i}."
        L = mtpx.TargetLayerWeights()
        L.attn_hc = d.hc(ck, p + "attn_hyper_connection", True)
        L.mlp_hc = d.hc(ck, p + "mlp_hyper_connection", True)
        if (i + 1) % TARGET["full_attention_interval"] == 0:
            L.kind = 1
            L.attn = d.attention(ck, p)
        else:
            L.kind = 0
            L.gdn = d.gdn(ck, p)
            L.attn.moe = d.moe(ck, p)
        if i == 1:
            L.ple = d.ple(ck, p + "ple.")
        layers.append(L)
    target = mtpx.Target.adopt(ctx, tc, tw, layers)
    m = t + "mtp."
    hw = mtpx.HeadWeights()
    hw.embed = tw.embed
    hw.pre_norm_embedding = d.put(ck[m + "pre_fc_norm_embedding.weight"])
    hw.pre_norm_hidden = d.put(ck[m + "pre_fc_norm_hidden.weight"])
    hw.fc_embedding = d.q4(ck, m + "fc_embedding")
    hw.fc_hidden = d.q4(ck, m + "fc_hidden")
    hw.final_hc = d.hc(ck, m + "hyper_connection_mixer", False)
    hw.attn_hc = d.hc(ck, m + "layers.0.attn_hyper_connection", True)
    hw.mlp_hc = d.hc(ck, m + "layers.0.mlp_hyper_connection", True)
    hw.layer = d.attention(ck, m + "layers.0.")
    V = TARGET["vocab"]
    low = 500 + (8 - (500 + (V - 980)) % 8) % 8
    ids = np.r_[np.arange(low), np.arange(980, V)].astype(np.int32)
    hw.shortlist = d.q4(ck, t + "lm_head", rows=ids)
    hw.shortlist_ids = d.put(ids)
    hw.shortlist_rows = len(ids)
    head = mtpx.MTPHead.adopt(ctx, hcfg, hw)
    return target, head, d


def _ngram_geometry():
    nh = (PLE["ngram_size"] - 1) * PLE["heads_per_ngram"]
    vocab = np.array(O.primes_above(PLE["vocab_base"], nh), np.int64)
    return vocab, np.concatenate([[0], np.cumsum(vocab)[:-1]]).astype(np.int64)


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def _outputs(ctx, t, head, windows):
    """Verify logits/multi of consecutive windows, then one head step over the last window's multi."""
    import mtpx
    st = mtpx.TargetState(ctx, t)
    V, W, H = TARGET["vocab"], TARGET["hc"] * LAYER["hidden"], LAYER["hidden"]
    out = []
    for ids in windows:
        lg = torch.zeros(len(ids), V, dtype=torch.bfloat16, device="cuda")
        mt = torch.zeros(len(ids), W, dtype=torch.bfloat16, device="cuda")
        t.verify(st, dev(np.asarray(ids, np.int32)), lg, mt)
        st.commit(len(ids))
        out += [host(lg), host(mt)]
    kv = mtpx.KVCache(ctx, LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"])
    mn = torch.zeros(len(windows[-1]), W, dtype=torch.bfloat16, device="cuda")
    sm = torch.zeros(len(windows[-1]), H, dtype=torch.bfloat16, device="cuda")
    dr = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    head.forward(kv, dev(np.asarray(windows[-1], np.int32)), dev(out[-1]), mn, sm, dr)
    out += [host(mn), host(sm), host(dr)]
    kv.close()
    st.close()
    return out


def test_loaded_equals_adopted_and_oracle(ctx, tmp_path):
    import mtpx
    from oracle.target_ref import download_target, oracle_verify
    tc, hcfg = _cfgs()
    vocab, offs = _ngram_geometry()
    ck = _make_checkpoint(71, vocab, offs)
    files = _write_checkpoint(tmp_path, ck)
    print("case checkpoint load", flush=True)
    cp = mtpx.Checkpoint(files)
    assert cp.count() == len(ck)
    lt = mtpx.Target.load(ctx, tc, cp)
    lh = mtpx.MTPHead.load(ctx, hcfg, cp, lt)
    cp.close()  # the loaded copies are on the device
    at, ah, keep = _adopt(ctx, tc, hcfg, ck)
    got_tab = lt.layer_weights(1).ple.table
    assert list(got_tab.vocab)[:len(vocab)] == list(vocab) and list(got_tab.offset)[:len(offs)] == list(offs)
    windows = [[5, 77, 7, 0, 981, 999], [123, 9], [42, 500, 3]]
    a, b = _outputs(ctx, lt, lh, windows), _outputs(ctx, at, ah, windows)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    print("case checkpoint oracle", flush=True)
    cfg = dict(LAYER, **TARGET, ple_layer=1)
    ow = download_target(lt, cfg)
    assert "sg_w" in ow["layers"][0]["moe"]
    HK, D, P, hc, H = LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"], TARGET["hc"], LAYER["hidden"]
    state = dict(kc={}, vc={}, conv={}, ssm={}, ple=(np.zeros((9, hc * H), np.uint16), np.array([7, 7], np.int32)))
    for i, L in enumerate(ow["layers"]):
        if L["kind"] == 1:
            state["kc"][i], state["vc"][i] = np.zeros((HK, P, D), np.uint16), np.zeros((HK, P, D), np.uint16)
        else:
            g = L["gdn"]["geom"]
            state["conv"][i], state["ssm"][i] = (np.zeros((g.kc - 1, g.conv_dim), np.uint16),
                                                 np.zeros((g.hv, 128, 128), np.float32))
    lg, mt, _, _ = oracle_verify(ow, cfg, state, np.asarray(windows[0], np.int32), 0)
    assert np.array_equal(a[0], lg) and np.array_equal(a[1], mt)
    # a session over the loaded model decodes as over the adopted one
    s1, s2 = mtpx.Session(ctx, lt, lh), mtpx.Session(ctx, at, ah)
    prompt = dev(np.random.default_rng(72).integers(0, TARGET["vocab"], 13).astype(np.int32))
    t1, t2 = [s1.prefill(prompt)], [s2.prefill(prompt)]
    for k in (2, 0, 3):
        t1 += s1.round(k)
        t2 += s2.round(k)
    assert t1 == t2
    s1.close()
    s2.close()
    for o in (lh, ah, lt, at):
        o.close()


def test_loader_refusals(ctx, tmp_path):
    import mtpx
    tc, hcfg = _cfgs()
    vocab, offs = _ngram_geometry()
    ck = _make_checkpoint(73, vocab, offs)
    missing = "language_model.model.layers.2.mlp.shared_expert_gate.scales"
    d1 = tmp_path / "a"
    d1.mkdir()
    with pytest.raises(mtpx.MtpxError, match="shared_expert_gate.scales is missing"):
        mtpx.Target.load(ctx, tc, mtpx.Checkpoint(_write_checkpoint(d1, ck, drop=missing)))
    d2 = tmp_path / "b"
    d2.mkdir()
    wrong = "language_model.model.layers.3.self_attn.k_proj.weight"
    with pytest.raises(mtpx.MtpxError, match="k_proj.weight is U32"):
        mtpx.Target.load(ctx, tc, mtpx.Checkpoint(_write_checkpoint(d2, ck, reshape=wrong)))
    d3 = tmp_path / "c"
    d3.mkdir()
    bad = _make_checkpoint(73, vocab + 2, offs)
    with pytest.raises(mtpx.MtpxError, match="n-gram head"):
        mtpx.Target.load(ctx, tc, mtpx.Checkpoint(_write_checkpoint(d3, bad)))
    d4 = tmp_path / "d"
    d4.mkdir()
    cp = mtpx.Checkpoint(_write_checkpoint(d4, ck, drop="language_model.mtp.fc_hidden.biases"))
    t = mtpx.Target.load(ctx, tc, cp)
    with pytest.raises(mtpx.MtpxError, match="fc_hidden.biases is missing"):
        mtpx.MTPHead.load(ctx, hcfg, cp, t)
    t.close()
    cp.close()
