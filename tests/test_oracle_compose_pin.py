"""Pins the oracle's compositions (oracle/layer_ref.py, oracle/head_ref.py,
oracle/target_ref.py) independently of the GPU and of their own code:

* float64 textbook forwards, written here from the reference's definitions -- the
  decoder layer (attention + MoE with pre-norm residuals), the MTP head step
  (Runner/Qwen4ExpMTP.swift:101-130, Runner/FastModel/TrackFastHead.swift:101-153) and a
  two-layer target stack, GDN then attention, each between hyper-connection mixers, then
  the final mixer and lm_head (Runner/FastModel/TrackFastModel.swift:1165-1265, 1330-1333)
  -- on dequantized weights, against the compositions within bf16 tolerance;
* exact reductions: with one hyper-connection stream, zero up and inject projections
  (every gate sigmoid(0) = 1/2, every inject weight 2 * sigmoid(0) = 1) and doubled norm
  scales, a target block is exactly the plain pre-norm layer x + sublayer(rms(x)) and the
  head step is exactly embedding/projection -> plain layer -> rms, bit for bit; a PLE
  block whose value projection and conv taps are zero adds nothing to the stream.

None of this imports the composition under test into the textbook side: the textbook
uses numpy only (dequantization s*q + b, RMS norm, RoPE, softmax, the delta rule)."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle.head_ref import oracle_head
from oracle.layer_ref import oracle_layer
from oracle.target_ref import oracle_commit, oracle_verify

H, HC, LW, E, K, F, GS = 256, 2, 64, 8, 2, 128, 32
HQ, HK, D, ROT, IDX, THETA, EPS = 4, 2, 64, 16, 32, 1e7, 1e-6
P, V = 32, 300
QW = 2 * HQ * D + 2 * HK * D + IDX


# ---------------------------------------------------------------------------- host weights
def bf(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def f(h):
    return O.bf16_to_f32(h).astype(np.float64)


def q4(r, rows, k, sigma=0.05):
    return O.affine_quantize(bf(r.standard_normal((rows, k)) * sigma), GS)


def zero_q4(rows, k):
    return (np.zeros((rows, k // 8), np.uint32), np.zeros((rows, k // GS), np.uint16),
            np.zeros((rows, k // GS), np.uint16))


def norm_w(r, n):
    return bf(1.0 + 0.1 * r.standard_normal(n))


def moe_w(r):
    w = {"router": bf(r.standard_normal((E, H)) * 0.3), "shared_gate": bf(r.standard_normal(H) * 0.05)}
    for n, (rows, k) in {"gate": (E * F, H), "up": (E * F, H), "down": (E * H, F),
                         "sh_gate": (F, H), "sh_up": (F, H), "sh_down": (H, F)}.items():
        w[n + "_w"], w[n + "_s"], w[n + "_b"] = q4(r, rows, k)
    return w


def attn_w(r):
    c, s = O.rope_table(P, ROT, THETA)
    return dict(attn_norm=norm_w(r, H), post_norm=norm_w(r, H), q_norm=norm_w(r, D), k_norm=norm_w(r, D),
                cos=c, sin=s, QW=QW, qkv=q4(r, QW, H), o=q4(r, H, HQ * D), moe=moe_w(r))


def hc_w(r, hc, inject=True):
    W = hc * H
    return dict(scale=norm_w(r, W), down=q4(r, LW, W), up=q4(r, W, LW, 0.5),
                inject=q4(r, hc, W) if inject else None)


def gdn_w(r):
    g = O.gdn_geom(1, 2, 4)
    return dict(in_proj=q4(r, g.proj_w, H), out_proj=q4(r, H, g.hv * 128),
                conv_w=bf(r.standard_normal((g.conv_dim, g.kc)) * 0.5),
                nea=-np.exp(r.standard_normal(g.hv) * 0.5).astype(np.float32), dtb=bf(r.standard_normal(g.hv)),
                nw=norm_w(r, 128), geom=g)


def cfg_of(hc):
    return dict(hidden=H, experts=E, top_k=K, expert_width=F, group_size=GS, heads=HQ, kv_heads=HK, head_dim=D,
                rot_dims=ROT, index_dim=IDX, rope_theta=THETA, eps=EPS, max_positions=P, hc=hc, lowrank=LW,
                vocab=V)


# ---------------------------------------------------------------------------- float64 textbook
def deq(t):
    wq, s, b = t
    q = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(wq.shape[0], -1)
    return q.astype(np.float64) * np.repeat(f(s), GS, 1) + np.repeat(f(b), GS, 1)


def rms(x, w):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + EPS) * w


def sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    return x * sig(x)


def t_hc_norm(resid, out, inj, scale, hc, tile=False):
    """stream = residual (tiled) + out (x) inject per stream; normed = per-stream rms * scale."""
    st = np.tile(resid, (1, hc)) if tile else resid.copy()
    if out is not None:
        st = st + np.concatenate([out * (1.0 if inj is None else inj[:, c:c + 1]) for c in range(hc)], 1)
    S = st.shape[0]
    n = rms(st.reshape(S, hc, H), f(scale).reshape(hc, H)).reshape(S, hc * H)
    return st, n


def t_mix(m, n, hc):
    w = silu(n @ deq(m["down"]).T) @ deq(m["up"]).T
    S = n.shape[0]
    x = (sig(w) * n).reshape(S, hc, H).sum(1)
    j = 2 * sig(n @ deq(m["inject"]).T) if m["inject"] is not None else None
    return x, j


def t_rope(v, pos):
    half = ROT // 2
    inv = THETA ** (-2.0 * np.arange(half) / ROT)
    ang = pos * inv
    c, s = np.cos(ang), np.sin(ang)
    o = v.copy()
    o[:half] = v[:half] * c - v[half:ROT] * s
    o[half:ROT] = v[half:ROT] * c + v[:half] * s
    return o


def t_attn(w, x, kc, vc, pos0):
    """qkv rows q | gate | k | v | index keys; q/k RMS norm then RoPE; causal softmax over the
    cache + window (GQA); output gated by sigmoid(gate); o_proj.  kc/vc (float64) receive the
    window's keys and values."""
    S = x.shape[0]
    qkv = x @ deq(w["qkv"]).T
    out = np.zeros((S, HQ * D))
    for s in range(S):
        for h in range(HK):
            k = qkv[s, 2 * HQ * D + h * D:2 * HQ * D + (h + 1) * D]
            kc[h, pos0 + s] = t_rope(rms(k, f(w["k_norm"])), pos0 + s)
            vc[h, pos0 + s] = qkv[s, 2 * HQ * D + HK * D + h * D:2 * HQ * D + HK * D + (h + 1) * D]
    for s in range(S):
        T = pos0 + s + 1
        for h in range(HQ):
            q = t_rope(rms(qkv[s, h * D:(h + 1) * D], f(w["q_norm"])), pos0 + s)
            kv = h // (HQ // HK)
            a = kc[kv, :T] @ q / np.sqrt(D)
            p = np.exp(a - a.max())
            p /= p.sum()
            out[s, h * D:(h + 1) * D] = (p @ vc[kv, :T]) * sig(qkv[s, HQ * D + h * D:HQ * D + (h + 1) * D])
    return out @ deq(w["o"]).T


def t_moe(w, x):
    R, SGt = f(w["router"]).reshape(E, H), f(w["shared_gate"])
    G, U, Dn = deq((w["gate_w"], w["gate_s"], w["gate_b"])), deq((w["up_w"], w["up_s"], w["up_b"])), \
        deq((w["down_w"], w["down_s"], w["down_b"]))
    SG, SU, SD = deq((w["sh_gate_w"], w["sh_gate_s"], w["sh_gate_b"])), \
        deq((w["sh_up_w"], w["sh_up_s"], w["sh_up_b"])), deq((w["sh_down_w"], w["sh_down_s"], w["sh_down_b"]))
    y = np.zeros_like(x)
    for m in range(x.shape[0]):
        lg = R @ x[m]
        order = np.argsort(-lg, kind="stable")[:K]
        p = np.exp(lg[order] - lg[order].max())
        p /= p.sum()
        for kk, e in enumerate(order):
            a = silu(G[e * F:(e + 1) * F] @ x[m]) * (U[e * F:(e + 1) * F] @ x[m])
            y[m] += p[kk] * (Dn[e * H:(e + 1) * H] @ a)
        y[m] += sig(SGt @ x[m]) * (SD @ (silu(SG @ x[m]) * (SU @ x[m])))
    return y


def t_gdn(w, x, conv, ssm):
    """Gated deltanet over the window: in_proj; per position the causal depthwise conv over the
    carried rows, SiLU, q = rms(q)/dk, k = rms(k)/sqrt(dk), beta = sigmoid(b),
    decay = exp(-exp(A_log) softplus(a + dt_bias)); S <- decay S; S += ((v - S k) beta) k^T;
    y = S q; out = norm_w * rms(y) * sigmoid(z); out_proj."""
    g = w["geom"]
    proj = x @ deq(w["in_proj"]).T
    rows = [r for r in conv]
    S_ = ssm.astype(np.float64).copy()
    cw = f(w["conv_w"])
    outs = []
    for t in range(x.shape[0]):
        rows.append(proj[t, :g.conv_dim])
        win = np.stack(rows[-g.kc:], 1)                       # [conv_dim, kc]
        xc = silu((win * cw).sum(1))
        beta = sig(proj[t, g.b_off:g.b_off + g.hv])
        decay = np.exp(w["nea"].astype(np.float64) * np.logaddexp(proj[t, g.a_off:g.a_off + g.hv] + f(w["dtb"]), 0))
        y = np.zeros(g.hv * 128)
        for h in range(g.hv):
            hk = h // (g.hv // g.hk)
            q = rms(xc[hk * 128:(hk + 1) * 128], 1.0) / 128
            k = rms(xc[(g.hk + hk) * 128:(g.hk + hk + 1) * 128], 1.0) / np.sqrt(128)
            v = xc[2 * g.hk * 128 + h * 128:2 * g.hk * 128 + (h + 1) * 128]
            S_[h] *= decay[h]
            S_[h] += np.outer((v - S_[h] @ k) * beta[h], k)
            yh = S_[h] @ q
            z = proj[t, g.z_off + h * 128:g.z_off + (h + 1) * 128]
            y[h * 128:(h + 1) * 128] = rms(yh, f(w["nw"])) * sig(z)
        outs.append(y)
    return np.array(outs) @ deq(w["out_proj"]).T


def relerr(got_bf16, ref):
    got = f(got_bf16).reshape(ref.shape)
    return np.linalg.norm(got - ref) / np.linalg.norm(ref)


# ---------------------------------------------------------------------------- textbook comparisons
def test_layer_matches_float64_textbook():
    r = np.random.default_rng(21)
    w = attn_w(r)
    cfg = cfg_of(1)
    pos0, S = 5, 3
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    vc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    K64, V64 = f(kc), f(vc)
    x = bf(r.standard_normal((S, H)))
    got = oracle_layer(w, cfg, kc, vc, x, pos0)
    X = f(x)
    s = X + t_attn(w, rms(X, f(w["attn_norm"])), K64, V64, pos0)
    ref = s + t_moe(w["moe"], rms(s, f(w["post_norm"])))
    assert relerr(got, ref) < 1e-2, relerr(got, ref)


def head_w(r, hc, zero_mix=False):
    w = dict(layer=attn_w(r), embed=q4(r, V, H, 1.0), pre_norm_embedding=norm_w(r, H),
             pre_norm_hidden=norm_w(r, hc * H), fc_embedding=q4(r, H, H), fc_hidden=q4(r, H, H))
    for name in ("attn_hc", "mlp_hc", "final_hc"):
        w[name] = hc_w(r, hc, inject=name != "final_hc")
        if zero_mix:
            w[name]["up"] = zero_q4(hc * H, LW)
            if w[name]["inject"] is not None:
                w[name]["inject"] = zero_q4(hc, hc * H)
    w["shortlist"] = q4(r, 64, H)
    w["shortlist_ids"] = np.arange(64, dtype=np.int32) * 3
    return w


def test_head_matches_float64_textbook():
    r = np.random.default_rng(22)
    w = head_w(r, HC)
    cfg = cfg_of(HC)
    pos0, S = 4, 3
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    vc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    K64, V64 = f(kc), f(vc)
    ids = np.array([3, 250, 17], np.int32)
    multi = bf(r.standard_normal((S, HC * H)))
    mn, sample, _ = oracle_head(w, cfg, kc, vc, ids, multi, pos0)
    # textbook: embed -> rms -> fc_embedding; multi -> rms over the flat row -> fc_hidden per stream
    e = deq(w["embed"])[ids]
    emb = rms(e, f(w["pre_norm_embedding"])) @ deq(w["fc_embedding"]).T
    hs = (rms(f(multi), f(w["pre_norm_hidden"])).reshape(S * HC, H) @ deq(w["fc_hidden"]).T).reshape(S, HC * H)
    hyper = hs + np.tile(emb, (1, HC))
    st, n = t_hc_norm(hyper, None, None, w["attn_hc"]["scale"], HC)
    x, j = t_mix(w["attn_hc"], n, HC)
    a = t_attn(w["layer"], x, K64, V64, pos0)
    st, n = t_hc_norm(st, a, j, w["mlp_hc"]["scale"], HC)
    x, j = t_mix(w["mlp_hc"], n, HC)
    m = t_moe(w["layer"]["moe"], x)
    st, n = t_hc_norm(st, m, j, w["final_hc"]["scale"], HC)
    smp, _ = t_mix(w["final_hc"], n, HC)
    assert relerr(mn, st) < 2e-2, relerr(mn, st)
    assert relerr(sample, smp) < 2e-2, relerr(sample, smp)


def target_w(r, hc, kinds, zero_mix=False, ple=None):
    layers = []
    for i, kind in enumerate(kinds):
        L = dict(kind=kind, attn_hc=hc_w(r, hc), mlp_hc=hc_w(r, hc))
        if kind == 1:
            L["attn"] = attn_w(r)
            L["moe"] = L["attn"]["moe"]
        else:
            L["gdn"] = gdn_w(r)
            L["moe"] = moe_w(r)
        if zero_mix:
            for name in ("attn_hc", "mlp_hc"):
                L[name]["up"] = zero_q4(hc * H, LW)
                L[name]["inject"] = zero_q4(hc, hc * H)
        layers.append(L)
    w = dict(embed=q4(r, V, H, 1.0), lm_head=q4(r, V, H), final_hc=hc_w(r, hc, inject=False), layers=layers)
    if zero_mix:
        w["final_hc"]["up"] = zero_q4(hc * H, LW)
    return w


def gdn_state(r, g):
    return bf(r.standard_normal((g.kc - 1, g.conv_dim))), (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(
        np.float32)


def test_target_two_layer_stack_matches_float64_textbook():
    r = np.random.default_rng(23)
    kinds = [0, 1]
    w = target_w(r, HC, kinds)
    cfg = dict(cfg_of(HC), key_heads=1, value_heads=2, conv_kernel=4)
    pos0 = 6
    conv, ssm = gdn_state(r, w["layers"][0]["gdn"]["geom"])
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    vc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    state = dict(kc={1: kc}, vc={1: vc}, conv={0: conv}, ssm={0: ssm})
    K64, V64 = f(kc), f(vc)
    ids = np.array([5, 299, 42, 7], np.int32)
    logits, multi, mixed, _ = oracle_verify(w, cfg, state, ids, pos0)
    # textbook stack: tiled embedding; per layer inject-norm, mixer, sublayer, inject-norm, mixer, MoE
    resid, out, inj, tile = deq(w["embed"])[ids], None, None, True
    for i, L in enumerate(w["layers"]):
        st, n = t_hc_norm(resid, out, inj, L["attn_hc"]["scale"], HC, tile)
        x, j = t_mix(L["attn_hc"], n, HC)
        a = t_gdn(L["gdn"], x, f(conv), ssm) if L["kind"] == 0 else t_attn(L["attn"], x, K64, V64, pos0)
        st, n = t_hc_norm(st, a, j, L["mlp_hc"]["scale"], HC)
        x, j = t_mix(L["mlp_hc"], n, HC)
        resid, out, inj, tile = st, t_moe(L["moe"], x), j, False
    mt, n = t_hc_norm(resid, out, inj, w["final_hc"]["scale"], HC)
    mx, _ = t_mix(w["final_hc"], n, HC)
    lg = mx @ deq(w["lm_head"]).T
    assert relerr(multi, mt) < 3e-2, relerr(multi, mt)
    assert relerr(mixed, mx) < 3e-2, relerr(mixed, mx)
    assert relerr(logits, lg) < 3e-2, relerr(logits, lg)


# ---------------------------------------------------------------------------- exact reductions
def _double(scale):
    return bf(2.0 * f(scale))  # exact in bf16


@pytest.mark.parametrize("kinds", [[1], [0], [0, 1]], ids=["attention", "gdn", "gdn+attention"])
def test_target_one_stream_reduces_to_plain_prenorm_layers(kinds):
    """hc = 1, zero up/inject: each block is s + sublayer(rms(s)) exactly; the final mixer is rms."""
    r = np.random.default_rng(24 + len(kinds))
    w = target_w(r, 1, kinds, zero_mix=True)
    cfg = dict(cfg_of(1), key_heads=1, value_heads=2, conv_kernel=4)
    pos0 = 3
    state, st2 = dict(kc={}, vc={}, conv={}, ssm={}), {}
    for i, k in enumerate(kinds):
        if k == 1:
            kc = np.zeros((HK, P, D), np.uint16)
            kc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
            vc = kc[::-1].copy()
            state["kc"][i], state["vc"][i] = kc, vc
            st2[i] = (kc.copy(), vc.copy())
        else:
            state["conv"][i], state["ssm"][i] = gdn_state(r, w["layers"][i]["gdn"]["geom"])
    ids = np.array([1, 2, 250], np.int32)
    # the plain stack: norm weights = the block scales halved (the mixer's gate 1/2 undone)
    norms = [(bf(0.5 * f(L["attn_hc"]["scale"])), bf(0.5 * f(L["mlp_hc"]["scale"]))) for L in w["layers"]]
    for L, (a, b) in zip(w["layers"], norms):
        L["attn_hc"]["scale"], L["mlp_hc"]["scale"] = _double(a), _double(b)
    fw = bf(0.5 * f(w["final_hc"]["scale"]))
    w["final_hc"]["scale"] = _double(fw)
    logits, multi, mixed, _ = oracle_verify(w, cfg, state, ids, pos0)
    x = O.embed_rows(*w["embed"], GS, ids)
    for i, (L, (na, nm)) in enumerate(zip(w["layers"], norms)):
        if L["kind"] == 1:
            kc, vc = st2[i]
            lw = dict(L["attn"], attn_norm=na, post_norm=nm)
            x = oracle_layer(lw, cfg, kc, vc, x, pos0)
        else:
            h = O.rmsnorm(x, na, EPS)
            d = L["gdn"]
            proj, _ = O.qmv(*d["in_proj"], GS, h)
            g = O.gdn_core(d["geom"], proj, state["conv"][i], state["ssm"][i], d["conv_w"], d["nea"], d["dtb"],
                           d["nw"], EPS)
            ao, _ = O.qmv(*d["out_proj"], GS, g["gated"])
            s = O.f32_to_bf16(O.bf16_to_f32(x) + O.bf16_to_f32(ao))
            m = O.moe_block(L["moe"], O.rmsnorm(s, nm, EPS), H, E, K, F, GS)["y"]
            x = O.f32_to_bf16(O.bf16_to_f32(s) + O.bf16_to_f32(m))
    assert np.array_equal(multi, x)
    assert np.array_equal(mixed, O.rmsnorm(x, fw, EPS))
    assert np.array_equal(logits, O.qmv(*w["lm_head"], GS, O.rmsnorm(x, fw, EPS))[0])


def test_head_one_stream_reduces_to_projections_and_plain_layer():
    r = np.random.default_rng(27)
    w = head_w(r, 1, zero_mix=True)
    cfg = cfg_of(1)
    na, nm, nf = norm_w(r, H), norm_w(r, H), norm_w(r, H)
    w["attn_hc"]["scale"], w["mlp_hc"]["scale"], w["final_hc"]["scale"] = _double(na), _double(nm), _double(nf)
    pos0, S = 2, 2
    kc = np.zeros((HK, P, D), np.uint16)
    kc[:, :pos0] = bf(r.standard_normal((HK, pos0, D)))
    vc = kc.copy()
    kc2, vc2 = kc.copy(), vc.copy()
    ids = np.array([9, 123], np.int32)
    multi = bf(r.standard_normal((S, H)))
    mn, sample, _ = oracle_head(w, cfg, kc, vc, ids, multi, pos0)
    e = O.embed_rows(*w["embed"], GS, ids)
    emb, _ = O.qmv(*w["fc_embedding"], GS, O.rmsnorm(e, w["pre_norm_embedding"], EPS))
    hs, _ = O.qmv(*w["fc_hidden"], GS, O.rmsnorm(multi, w["pre_norm_hidden"], EPS))
    hyper = O.f32_to_bf16(O.bf16_to_f32(hs) + O.bf16_to_f32(emb))
    lw = dict(w["layer"], attn_norm=na, post_norm=nm)
    s2 = oracle_layer(lw, cfg, kc2, vc2, hyper, pos0)
    assert np.array_equal(mn, s2)
    assert np.array_equal(sample, O.rmsnorm(s2, nf, EPS))


def test_zero_ple_block_adds_nothing():
    """A PLE block with zero value projection and zero conv taps: gated = sigmoid(g) * 0 = 0 and the
    conv of zero taps is 0, so the stream passes unchanged and the re-norm equals the plain norm:
    the verify with that block on layer 0 equals the verify without it, bit for bit."""
    from oracle.target_ref import ple_cfg_dict  # noqa: F401  (the dict layout the composition reads)
    r = np.random.default_rng(28)
    kinds = [0, 1]
    w = target_w(r, HC, kinds)
    cfg = dict(cfg_of(HC), key_heads=1, value_heads=2, conv_kernel=4)
    conv, ssm = gdn_state(r, w["layers"][0]["gdn"]["geom"])
    kc = np.zeros((HK, P, D), np.uint16)
    kc[:, :2] = bf(r.standard_normal((HK, 2, D)))
    ids = np.array([4, 5], np.int32)

    def state():
        return dict(kc={1: kc.copy()}, vc={1: kc[::-1].copy()}, conv={0: conv.copy()}, ssm={0: ssm.copy()},
                    ple=(bf(r.standard_normal((9, HC * H))), np.array([1, 2], np.int32)))

    base = oracle_verify(w, cfg, state(), ids, 2)
    nh, rd = 4, 64
    table = O.affine_quantize(bf(r.standard_normal((50, rd))), 32)
    vocab = np.array(O.primes_above(10, nh), np.int64)
    ple = dict(key_proj=q4(r, HC * H, nh * rd), value_proj=zero_q4(H, nh * rd), norm_key=norm_w(r, HC * H),
               norm_query=norm_w(r, HC * H), norm_conv=norm_w(r, HC * H),
               conv_w=np.zeros((HC * H, 4), np.uint16), table=table, mult=np.array([1, 3, 5], np.int64),
               vocab=vocab, offs=np.concatenate([[0], np.cumsum(vocab)[:-1]]).astype(np.int64))
    w["layers"][0]["ple"] = ple
    w["layers"][0]["ple_cfg"] = dict(hidden=H, hc=HC, embed_dim=nh * rd, ngram_size=3, heads_per_ngram=2,
                                     conv_kernel=4, group_size=GS, row_group_size=32, eos=0, eps=EPS)
    with_ple = oracle_verify(w, cfg, state(), ids, 2)
    for a, b in zip(base[:3], with_ple[:3]):
        assert np.array_equal(a, b)


def test_commit_replays_the_kept_positions():
    """oracle_commit(n) leaves the GDN state a verify of exactly the first n positions leaves."""
    r = np.random.default_rng(29)
    w = target_w(r, HC, [0, 1])
    cfg = dict(cfg_of(HC), key_heads=1, value_heads=2, conv_kernel=4)
    conv, ssm = gdn_state(r, w["layers"][0]["gdn"]["geom"])
    kc = np.zeros((HK, P, D), np.uint16)

    def state():
        return dict(kc={1: kc.copy()}, vc={1: kc.copy()}, conv={0: conv.copy()}, ssm={0: ssm.copy()})

    ids = np.array([7, 8, 9, 10], np.int32)
    s1 = state()
    win = oracle_verify(w, cfg, s1, ids, 0)[3]
    oracle_commit(w, cfg, s1, win, 2)
    s2 = state()
    oracle_verify(w, cfg, s2, ids[:2], 0)
    d = w["layers"][0]["gdn"]
    g = O.gdn_core(d["geom"], oracle_verify(w, cfg, state(), ids[:2], 0)[3][0], conv, ssm, d["conv_w"], d["nea"],
                   d["dtb"], d["nw"], EPS)
    assert np.array_equal(s1["ssm"][0], g["ssm"]) and np.array_equal(s1["conv"][0], g["conv_state"])
