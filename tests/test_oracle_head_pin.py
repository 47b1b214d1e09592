"""Pins the oracle's MTP-head pieces (embedding rows, hyper-connection norm and
mixer, shortlist argmax) independently of the GPU: float64 brute force, torch's
bf16 arithmetic, exact special cases and invariants.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def rng(seed=0):
    return np.random.default_rng(seed)


def bf16(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


def f32(h):
    return O.bf16_to_f32(h)


def tbf(h):
    """bf16 bit patterns -> torch bfloat16 tensor (torch does bf16 ops with one rounding each)."""
    return torch.from_numpy(np.asarray(h, np.uint16).astype(np.int16)).view(torch.bfloat16)


def tbits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------- embedding rows
@pytest.mark.parametrize("gs", [32, 64])
def test_embed_rows_match_torch_bf16_dequant(gs):
    # MLX affine_dequantize in bf16: bf16(bf16(scale * q) + bias); torch's bf16 ops round each step
    r = rng(gs)
    V, H = 40, 256
    w = bf16(r.standard_normal((V, H)) * 0.05)
    wq, s, b = O.affine_quantize(w, gs)
    ids = np.array([7, 0, 39, 7, 12], np.int32)
    got = O.embed_rows(wq, s, b, gs, ids)
    q = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(V, H).astype(np.float32)
    qt = torch.from_numpy(q).to(torch.bfloat16)  # 0..15 exact in bf16
    st = tbf(np.repeat(s, gs, axis=1))
    bt = tbf(np.repeat(b, gs, axis=1))
    want = tbits(st * qt + bt)
    assert np.array_equal(got, want[ids])
    # within a quantisation step of the source weights
    step = np.repeat(f32(s), gs, axis=1)
    assert np.all(np.abs(f32(got) - f32(w)[ids]) <= 1.01 * np.abs(step[ids]) + 2e-3)


# ---------------------------------------------------------------------------- hc norm
def test_hc_norm_plain_matches_float64_rms():
    r = rng(3)
    S, hc, H = 3, 4, 512
    x = bf16(r.standard_normal((S, hc * H)) * 2.0)
    scale = bf16(1.0 + 0.1 * r.standard_normal(hc * H))
    stream, normed = O.hc_norm(x, None, None, scale, hc, 1e-6)
    assert np.array_equal(stream, x)
    xg = f32(x).astype(np.float64).reshape(S, hc, H)
    ref = xg / np.sqrt((xg ** 2).mean(-1, keepdims=True) + 1e-6) * f32(scale).reshape(hc, H)
    got = f32(normed).astype(np.float64).reshape(S, hc, H)
    assert np.all(np.abs(got - ref) <= 2 ** -6 * np.abs(ref) + 1e-6)  # two bf16 roundings


def test_hc_norm_inject_stream_matches_torch():
    r = rng(4)
    S, hc, H = 2, 4, 256
    res = bf16(r.standard_normal((S, hc * H)))
    out = bf16(r.standard_normal((S, H)))
    inj = bf16(r.standard_normal((S, hc)))
    scale = bf16(np.full(hc * H, 0.25))
    stream, _ = O.hc_norm(res, out, inj, scale, hc, 1e-6)
    rt, ot, it = tbf(res).reshape(S, hc, H), tbf(out).reshape(S, 1, H), tbf(inj).reshape(S, hc, 1)
    want = tbits(rt + ot * it).reshape(S, hc * H)
    assert np.array_equal(stream, want)
    # add-only mode: one bf16 rounding of residual + out for every stream
    stream2, _ = O.hc_norm(res, out, None, scale, hc, 1e-6)
    assert np.array_equal(stream2, tbits(rt + ot).reshape(S, hc * H))


def test_hc_norm_tile_equals_replicated_and_scale_is_linear():
    r = rng(5)
    S, hc, H = 2, 4, 256
    x = bf16(r.standard_normal((S, H)))
    scale = bf16(r.uniform(0.5, 1.5, hc * H))
    st_t, n_t = O.hc_norm(x, None, None, scale, hc, 1e-6, tile=True)
    rep = np.tile(x, (1, hc))
    st_r, n_r = O.hc_norm(rep, None, None, scale, hc, 1e-6)
    assert np.array_equal(st_t, st_r) and np.array_equal(n_t, n_r)
    _, n2 = O.hc_norm(rep, None, None, bf16(2.0 * f32(scale)), hc, 1e-6)
    assert np.array_equal(f32(n2), 2.0 * f32(n_r))  # doubling is exact in bf16


def test_hc_norm_one_group_is_rmsnorm():
    r = rng(6)
    x = bf16(r.standard_normal((3, 1024)))
    w = bf16(1.0 + 0.1 * r.standard_normal(1024))
    _, n = O.hc_norm(x, None, None, w, 1, 1e-6)
    assert np.array_equal(n, O.rmsnorm(x, w, 1e-6))


# ---------------------------------------------------------------------------- mixer
def test_hc_mix_saturated_gates_and_inject():
    r = rng(7)
    S, hc, H = 2, 4, 128
    normed = bf16(r.standard_normal((S, hc * H)))
    inj = bf16(np.zeros((S, hc)))
    # sigmoid(40) == 1 in bf16: input = running bf16 sum of the streams (torch, stream order)
    x, j = O.hc_mix(bf16(np.full((S, hc * H), 40.0)), normed, inj, hc)
    acc = torch.zeros(S, H, dtype=torch.bfloat16)
    nt = tbf(normed).reshape(S, hc, H)
    for c in range(hc):
        acc = acc + nt[:, c]
    assert np.array_equal(x, tbits(acc))
    assert np.all(f32(j) == 1.0)  # 2 * sigmoid(0)
    # sigmoid(-40) underflows to ~0: the input vanishes
    x0, _ = O.hc_mix(bf16(np.full((S, hc * H), -40.0)), normed, None, hc)
    assert np.all(np.abs(f32(x0)) < 1e-12)


def test_hc_mix_matches_float64():
    r = rng(8)
    S, hc, H = 3, 4, 256
    w = bf16(r.standard_normal((S, hc * H)) * 2)
    n = bf16(r.standard_normal((S, hc * H)))
    x, _ = O.hc_mix(w, n, None, hc)
    sig = 1.0 / (1.0 + np.exp(-f32(w).astype(np.float64)))
    ref = (sig * f32(n)).reshape(S, hc, H).sum(1)
    scale = np.abs(f32(n)).reshape(S, hc, H).sum(1)
    assert np.all(np.abs(f32(x) - ref) <= 2 ** -6 * scale + 1e-6)


def test_silu_rows_is_scalar_silu():
    x = bf16(np.linspace(-8, 8, 513))
    y = O.silu_rows(x)
    assert np.array_equal(y, bf16([O.lib().o_silu_bf16(float(v)) for v in f32(x)]))


# ---------------------------------------------------------------------------- shortlist
def test_shortlist_argmax_ties_and_mapping():
    ids = np.array([0, 1, 2, 3, 1000, 1001], np.int32)
    y = bf16([0.5, 2.0, 1.0, 2.0, -3.0, 2.0])
    assert O.shortlist_argmax(y, ids) == 1  # lowest position among the equal maxima
    y2 = bf16([0.5, 1.0, 1.0, 1.0, 1.5, 1.5])
    assert O.shortlist_argmax(y2, ids) == 1000
    # values equal only after bf16 rounding count as ties
    y3 = bf16([1.0, 1.0 + 2 ** -10, 0, 0, 0, 0])
    assert O.shortlist_argmax(y3, ids) == 0
