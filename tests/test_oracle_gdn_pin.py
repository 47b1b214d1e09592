"""Pins the oracle's gated-deltanet sublayer (o_gdn_*) independently of the GPU:
float64 restatements of the prep (conv, SiLU, q/k RMS norm, gates), the delta
rule, the gated RMS norm; the zero-state closed form; special values of the
scalar helpers; and window-split invariance of the sequential composition.
"""
import numpy as np
import pytest

from oracle import oracle as O


def bf(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def f(h):
    return O.bf16_to_f32(h).astype(np.float64)


def ulp32(x):
    x = np.abs(np.asarray(x, np.float32))
    return np.spacing(x).astype(np.float64)


def make(seed, hk=2, hv=6, S=3, state_scale=0.1):
    r = np.random.default_rng(seed)
    g = O.gdn_geom(hk, hv)
    w = dict(
        proj=bf(r.standard_normal((S, g.proj_w))),
        cs=bf(r.standard_normal((3, g.conv_dim))),
        ssm=(r.standard_normal((hv, 128, 128)) * state_scale).astype(np.float32),
        cw=bf(r.standard_normal((g.conv_dim, 4)) * 0.5),
        nea=-np.exp(r.standard_normal(hv) * 0.5).astype(np.float32),
        dtb=bf(r.standard_normal(hv)),
        nw=bf(1 + 0.1 * r.standard_normal(128)),
    )
    return g, w


def run(g, w, proj=None, cs=None, ssm=None):
    return O.gdn_core(g, w["proj"] if proj is None else proj, w["cs"] if cs is None else cs,
                      w["ssm"] if ssm is None else ssm, w["cw"], w["nea"], w["dtb"], w["nw"])


# ---------------------------------------------------------------------------- scalar helpers
def test_log1p_det_within_two_ulp():
    L = O.lib()
    ys = np.concatenate([np.linspace(0, 1, 20001, dtype=np.float32), np.float32(2.0) ** -np.arange(1, 60)])
    got = np.array([L.o_log1p_det(float(y)) for y in ys], np.float64)
    ref = np.log1p(ys.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 2 * ulp32(ref) + 1e-45)
    assert L.o_log1p_det(0.0) == 0.0


def test_logaddexp0_bf16_matches_softplus():
    L = O.lib()
    xs = f(bf(np.linspace(-30, 30, 4001)))
    got = np.array([L.o_logaddexp0_bf16(float(x)) for x in xs])
    ref = np.logaddexp(xs, 0.0)
    # four bf16 roundings (difference exact, exp, log1p, sum): within 3 bf16 ulp of the value
    assert np.all(np.abs(got - ref) <= 3 * 2.0 ** -8 * np.maximum(ref, 2.0 ** -126) + 1e-30)
    assert np.array_equal(bf(got), bf(got).astype(np.uint16))  # results are bf16 values
    assert L.o_logaddexp0_bf16(float("inf")) == float("inf")
    assert L.o_logaddexp0_bf16(float("-inf")) == 0.0
    assert np.isnan(L.o_logaddexp0_bf16(float("nan")))
    assert L.o_logaddexp0_bf16(0.0) == f(bf(np.log(2.0)))[()]


def test_sigmoid_f32_matches_float64():
    L = O.lib()
    xs = np.linspace(-40, 40, 8001, dtype=np.float32)
    got = np.array([L.o_sigmoid_f32(float(x)) for x in xs], np.float64)
    ref = 1.0 / (1.0 + np.exp(-xs.astype(np.float64)))
    assert np.all(np.abs(got - ref) <= 4 * ulp32(ref) + 1e-7 * (xs > 0))


# ---------------------------------------------------------------------------- prep
def test_prep_matches_float64():
    g, w = make(1, S=1)
    o = run(g, w)
    cw, cs, prow = f(w["cw"]), f(w["cs"]), f(w["proj"][0])
    win = np.concatenate([cs, prow[None, :g.conv_dim]], 0)           # [4, CD]
    conv = (win.T * cw).sum(1)                                         # [CD]
    L = O.lib()
    # the bf16 SiLU is pinned on its own (tests/test_oracle_pin.py); the rest is float64 here
    x = np.array([L.o_silu_bf16(float(c)) for c in f(bf(conv))], np.float64)
    D = 128
    for vec in range(2 * g.hk):
        xs = x[vec * D:(vec + 1) * D]
        n = xs / np.sqrt((xs * xs).mean() + 1e-6)
        mul = 1 / 128 if vec < g.hk else 1 / np.sqrt(128)
        ref = mul * n
        got = f(o["q"][0, vec * D:(vec + 1) * D] if vec < g.hk else o["k"][0, (vec - g.hk) * D:(vec - g.hk + 1) * D])
        assert np.all(np.abs(got - ref) <= 2 ** -6 * np.abs(ref) + 1e-6), vec
    xv = x[2 * g.hk * D:]
    assert np.array_equal(f(o["v"][0]), xv)
    b = prow[g.b_off:g.b_off + g.hv]
    a = prow[g.a_off:g.a_off + g.hv]
    beta = 1 / (1 + np.exp(-b))
    assert np.all(np.abs(o["beta"][0] - beta) <= 2 ** -6 * beta + 1e-6)  # four bf16 roundings
    sp = np.logaddexp(a + f(w["dtb"]), 0)
    decay = np.exp(w["nea"].astype(np.float64) * sp)
    assert np.all(np.abs(o["decay"][0] - decay) <= 0.03 * decay + 1e-6)


def test_prep_conv_uses_state_then_window():
    # conv state rows shift by one per position: position 1 of a 2-window equals position 0
    # of a 1-window whose state holds the last 3 inputs
    g, w = make(2, S=2)
    o2 = run(g, w)
    cs1 = np.concatenate([w["cs"][1:], w["proj"][:1, :g.conv_dim]], 0)
    o1 = run(g, w, proj=w["proj"][1:], cs=cs1, ssm=o2["ssm"] * 0 + run(g, w, proj=w["proj"][:1])["ssm"])
    for key in ("q", "k", "v", "decay", "beta", "gated"):
        assert np.array_equal(o2[key][1], o1[key][0]), key
    assert np.array_equal(o2["conv_state"], o1["conv_state"])
    assert np.array_equal(o2["conv_state"][-1], w["proj"][1, :g.conv_dim])


# ---------------------------------------------------------------------------- recurrence
def test_delta_rule_matches_float64():
    g, w = make(3, S=4)
    o = run(g, w)
    ratio = g.hv // g.hk
    s = w["ssm"].astype(np.float64).copy()
    for t in range(4):
        for h in range(g.hv):
            hk = h // ratio
            q = f(o["q"][t, hk * 128:(hk + 1) * 128])
            k = f(o["k"][t, hk * 128:(hk + 1) * 128])
            v = f(o["v"][t, h * 128:(h + 1) * 128])
            s[h] *= o["decay"][t, h]
            kv = s[h] @ k
            delta = (v - kv) * o["beta"][t, h]
            s[h] += np.outer(delta, k)
            y = s[h] @ q
            got = f(o["y"][t, h * 128:(h + 1) * 128])
            scale = np.abs(s[h]) @ np.abs(q)
            assert np.all(np.abs(got - y) <= 2 ** -8 * np.abs(y) + 1e-5 * scale + 1e-6), (t, h)
    assert np.all(np.abs(o["ssm"] - s) <= 1e-5 * np.abs(s) + 1e-6)


def test_delta_rule_zero_state_closed_form():
    # from a zero state: kv = 0, delta = v * beta, S = delta k^T, y = (k . q) delta
    g, w = make(4, S=1)
    o = run(g, w, ssm=np.zeros_like(w["ssm"]))
    ratio = g.hv // g.hk
    for h in range(g.hv):
        hk = h // ratio
        q = f(o["q"][0, hk * 128:(hk + 1) * 128])
        k = f(o["k"][0, hk * 128:(hk + 1) * 128])
        v = f(o["v"][0, h * 128:(h + 1) * 128])
        delta = v * np.float64(o["beta"][0, h])
        assert np.allclose(o["delta"][0, h * 128:(h + 1) * 128], delta, rtol=1e-6, atol=0)
        y = (k @ q) * delta
        got = f(o["y"][0, h * 128:(h + 1) * 128])
        assert np.all(np.abs(got - y) <= 2 ** -8 * np.abs(y) + 1e-6 * np.abs(delta) * (np.abs(k) @ np.abs(q)))


def test_unit_decay_zero_beta_leaves_state():
    # decay == 1 (A_log -> -inf) and beta == 0: the state is untouched; y = S q
    g, w = make(5, S=1)
    w = dict(w, nea=np.zeros(g.hv, np.float32))
    proj = w["proj"].copy()
    proj[:, g.b_off:g.b_off + g.hv] = bf(np.full(g.hv, -200.0))  # sigmoid_bf16(-200) == 0
    o = run(g, w, proj=proj)
    assert np.all(o["decay"] == 1.0) and np.all(o["beta"] == 0.0)
    assert np.array_equal(o["ssm"], w["ssm"])


# ---------------------------------------------------------------------------- gated RMS
def test_gated_rms_matches_float64():
    g, w = make(6, S=2)
    o = run(g, w)
    nw = f(w["nw"])
    for t in range(2):
        for h in range(g.hv):
            y = f(o["y"][t, h * 128:(h + 1) * 128])
            z = f(w["proj"][t, g.z_off + h * 128:g.z_off + (h + 1) * 128])
            ref = nw * y / np.sqrt((y * y).mean() + 1e-6) / (1 + np.exp(-z))
            got = f(o["gated"][t, h * 128:(h + 1) * 128])
            assert np.all(np.abs(got - ref) <= 2 ** -6 * np.abs(ref) + 1e-6), (t, h)


# ---------------------------------------------------------------------------- composition
@pytest.mark.parametrize("split", [1, 2, 3])
def test_window_split_invariance(split):
    g, w = make(7, S=4)
    whole = run(g, w)
    a = run(g, w, proj=w["proj"][:split])
    b = run(g, w, proj=w["proj"][split:], cs=a["conv_state"], ssm=a["ssm"])
    assert np.array_equal(np.concatenate([a["gated"], b["gated"]]), whole["gated"])
    assert np.array_equal(b["ssm"], whole["ssm"])
    assert np.array_equal(b["conv_state"], whole["conv_state"])
