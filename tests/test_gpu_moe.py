"""GPU parity of the MoE block (router, top-k, expert-grouped gate|up + SwiGLU,
down + combine) against the oracle: routed ids, weights, logits and the FFN
output bit-exact.  Config 1 of BASELINE.json (H 2048, 64 experts, top-8 + shared,
F 768, gs 64, M in {1, 4}) and the full expert shapes (H 2560, top-10, F 640) with
a reduced expert count, at gs 32 and 64."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16  # noqa: E402

NAMES = ["router", "shared_gate", "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s",
         "down_b", "sh_gate_w", "sh_gate_s", "sh_gate_b", "sh_up_w", "sh_up_s", "sh_up_b", "sh_down_w",
         "sh_down_s", "sh_down_b"]


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def make_moe(seed, H, E, K, F, gs):
    """Seeded N(0, 0.02) bf16 weights quantised to MLX affine 4-bit (the config-1 recipe)."""
    r = np.random.default_rng(seed)

    def q(rows, k):
        return O.affine_quantize(rand_bf16(r, (rows, k), 0.02), gs)
    w = {}
    w["router"] = rand_bf16(r, (E, H), 0.02)
    w["shared_gate"] = rand_bf16(r, (H,), 0.02)
    for name, (rows, k) in {"gate": (E * F, H), "up": (E * F, H), "down": (E * H, F),
                            "sh_gate": (F, H), "sh_up": (F, H), "sh_down": (H, F)}.items():
        w[name + "_w"], w[name + "_s"], w[name + "_b"] = q(rows, k)
    return w


def run_case(ctx, w, H, E, K, F, gs, M, xseed, packed=False):
    import mtpx
    r = np.random.default_rng(xseed)
    x = rand_bf16(r, (M, H), 1.0)
    ref = O.moe_block(w, x, H, E, K, F, gs)
    dw = {n: dev(w[n]) for n in NAMES if n in w}
    if "sg_w" in w:  # the q4 shared-expert gate row (its packed pair row with the packed layout)
        dw["shared_gate_w"], dw["shared_gate_s"], dw["shared_gate_b"] = (dev(w["sg_w"]), dev(w["sg_s"]),
                                                                       dev(w["sg_b"]))
        if packed:
            dw["shared_gate_sb"] = ctx.pack_sb(dw["shared_gate_s"], dw["shared_gate_b"], H, gs)
    if packed:  # packed (scale, bias) rows for the expert GEMVs
        for n, Kd in (("gate", H), ("up", H), ("down", F), ("sh_gate", H), ("sh_up", H), ("sh_down", F)):
            dw[n + "_sb"] = ctx.pack_sb(dw[n + "_s"], dw[n + "_b"], Kd, gs)
    mw = mtpx.moe_weights_from(dw, H, E, K, F, gs)
    y = empty_bf16(M, H)
    idx = torch.zeros(M, K, dtype=torch.int32, device="cuda")
    wt = torch.zeros(M, K, dtype=torch.float32, device="cuda")
    lg = torch.zeros(M, E, dtype=torch.float32, device="cuda")
    nu = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.moe_forward(mw, dev(x), y, idx, wt, lg, nu)
    ctx.synchronize()
    assert np.array_equal(host(lg).view(np.uint32), ref["logits"].view(np.uint32))
    assert np.array_equal(host(idx), ref["idx"])
    assert np.array_equal(host(wt).view(np.uint32), ref["w"].view(np.uint32))
    assert int(host(nu)[0]) == len(np.unique(ref["idx"]))
    got = host(y)
    assert np.array_equal(got, ref["y"]), np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(ref["y"])).max()
    nbytes, n_unique = ctx.last_moe_bytes()
    assert n_unique == len(np.unique(ref["idx"]))
    B = lambda N, Kd: N * Kd // 2 + 4 * N * Kd // gs
    assert nbytes == (n_unique + 1) * (2 * B(F, H) + B(H, F)) + 2 * E * H + 2 * H
    return ref


@pytest.mark.parametrize("M,packed", [(1, False), (4, False), (4, True)])
def test_moe_config1_bit_exact(ctx, M, packed):
    print("case config1 M", M, "packed", packed, flush=True)
    H, E, K, F, gs = 2048, 64, 8, 768, 64
    w = make_moe(0x5EED0001, H, E, K, F, gs)
    run_case(ctx, w, H, E, K, F, gs, M, 0x5EED0002 + M, packed)


@pytest.mark.parametrize("gs,M,packed", [(64, 1, False), (64, 4, True), (64, 6, True), (32, 2, False), (32, 3, True),
                                         (32, 8, True)])
def test_moe_full_expert_shapes_bit_exact(ctx, gs, M, packed):
    print("case fullshape gs", gs, "M", M, "packed", packed, flush=True)
    H, E, K, F = 2560, 24, 10, 640
    w = make_moe(1000 + gs, H, E, K, F, gs)
    run_case(ctx, w, H, E, K, F, gs, M, 77 + M, packed)


@pytest.mark.parametrize("H,gs,M,packed", [(2560, 32, 4, True), (2560, 64, 1, False), (2560, 32, 8, False),
                                           (2048, 64, 3, True), (512, 32, 2, True)])
def test_moe_q4_shared_gate_bit_exact(ctx, H, gs, M, packed):
    """The checkpoint's shared-expert gate as a q4 row (mlp.shared_expert_gate): the router launch's
    extra workgroup computes it with the GEMV's lane rule; bit-exact against the oracle, with the
    packed pair row or the checkpoint's scales and biases, at the model's hidden size and others."""
    print("case moe q4 shared gate H", H, "gs", gs, "M", M, "packed", packed, flush=True)
    E, K, F = 24, 10 if H == 2560 else 4, 640 if H == 2560 else 256
    w = make_moe(3000 + H + gs, H, E, K, F, gs)
    r = np.random.default_rng(H + M)
    w["sg_w"], w["sg_s"], w["sg_b"] = O.affine_quantize(rand_bf16(r, (1, H), 0.3), gs)
    del w["shared_gate"]
    ref = run_case(ctx, w, H, E, K, F, gs, M, 91 + M, packed)
    gq, _ = O.qmv(w["sg_w"], w["sg_s"], w["sg_b"], gs, rand_bf16(np.random.default_rng(91 + M), (M, H), 1.0))
    assert np.array_equal(ref["gate"], gq[:, 0])


def test_moe_nan_token_routes_distinct_experts(ctx):
    """A token whose hidden state is NaN has NaN router logits: they rank as -inf, so the token
    still takes K distinct experts (the lowest indices) and the dispatch stays a permutation of the
    slots; the other tokens of the window are unaffected (bit-exact against the oracle)."""
    import mtpx
    print("case moe nan token", flush=True)
    H, E, K, F, gs, M = 2560, 24, 10, 640, 64, 4
    w = make_moe(1064, H, E, K, F, gs)
    x = rand_bf16(np.random.default_rng(81), (M, H), 1.0)
    x[1] = 0x7FC0  # bf16 NaN row
    ref = O.moe_block(w, x, H, E, K, F, gs)
    dw = {n: dev(w[n]) for n in NAMES}
    mw = mtpx.moe_weights_from(dw, H, E, K, F, gs)
    y = empty_bf16(M, H)
    idx = torch.zeros(M, K, dtype=torch.int32, device="cuda")
    ctx.moe_forward(mw, dev(x), y, idx)
    ctx.synchronize()
    got = host(idx)
    assert np.array_equal(got, ref["idx"])
    assert list(got[1]) == list(range(K))
    assert all(len(set(row)) == K for row in got)
    ok = [0, 2, 3]
    assert np.array_equal(host(y)[ok], ref["y"][ok])


def test_moe_router_ties_lowest_index(ctx):
    print("case router ties", flush=True)
    H, E, K, F, gs = 256, 16, 4, 64, 32
    w = make_moe(5, H, E, K, F, gs)
    # identical router rows 3, 9, 12 -> identical logits; lower index must win
    w["router"][9] = w["router"][3]
    w["router"][12] = w["router"][3]
    ref = run_case(ctx, w, H, E, K, F, gs, 3, 9)
    for m in range(3):
        sel = list(ref["idx"][m])
        for a, b in ((3, 9), (9, 12), (3, 12)):
            if b in sel:
                assert a in sel and sel.index(a) < sel.index(b)


@pytest.mark.parametrize("E", [512, 1024])
def test_moe_router_ties_within_and_across_lanes(ctx, E):
    """Equal logits among the leaders: copies of one router row on experts that share a lane of the
    route's wave (5, 69, 133, ... : expert mod 64 equal) and on neighbouring lanes (7, 8, 71), so the
    ranks take them in index order whether the tie is inside a lane's list or between lanes; a zero
    token has every logit +0 (all tied: experts 0..K-1 in order).  E 1024 holds 16 experts per lane."""
    print("case router lane ties E", E, flush=True)
    H, K, F, gs, M = 256, 10, 64, 32, 4
    w = make_moe(70 + E, H, E, K, F, gs)
    r = w["router"].reshape(E, H)
    r7 = O.bf16_to_f32(r[7])
    b5, b7 = O.f32_to_bf16((r7 * 4.0).astype(np.float32)), O.f32_to_bf16((r7 * 8.0).astype(np.float32))
    for e in [5, 69, 133, 261] + ([581, 965] if E > 512 else []):
        r[e] = b5
    for e in (7, 8, 71):
        r[e] = b7
    xr = np.random.default_rng(71)
    x = rand_bf16(xr, (M, H), 1.0)
    x[1] = 0
    x[2] = O.f32_to_bf16((r7 * 50.0).astype(np.float32))  # along row 7: both groups lead, group 7 first
    import mtpx
    ref = O.moe_block(w, x, H, E, K, F, gs)
    dw = {n: dev(w[n]) for n in NAMES}
    mw = mtpx.moe_weights_from(dw, H, E, K, F, gs)
    y = empty_bf16(M, H)
    idx = torch.zeros(M, K, dtype=torch.int32, device="cuda")
    wt = torch.zeros(M, K, dtype=torch.float32, device="cuda")
    ctx.moe_forward(mw, dev(x), y, idx, wt)
    ctx.synchronize()
    got = host(idx)
    assert np.array_equal(got, ref["idx"])
    assert np.array_equal(host(wt).view(np.uint32), ref["w"].view(np.uint32))
    assert np.array_equal(host(y), ref["y"])
    assert list(got[1]) == list(range(K))
    g5 = [5, 69, 133, 261] + ([581, 965] if E > 512 else [])
    lead = [7, 8, 71] + g5
    assert list(got[2][:len(lead)]) == lead


def test_moe_back_to_back_windows_route_their_own_logits():
    """One-window launches hand the router logits to the route through a per-context buffer that each
    route puts back to its sentinel: windows enqueued back to back on a fresh context (different
    tokens, widths and expert counts, no synchronisation between them) each route their own logits."""
    print("case back-to-back routes", flush=True)
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    try:
        H, K, F, gs = 256, 10, 64, 32
        runs = []
        for i, (E, M) in enumerate([(512, 4), (512, 4), (1024, 8), (512, 2), (1024, 1), (512, 8)]):
            w = make_moe(90 + E, H, E, K, F, gs)
            x = rand_bf16(np.random.default_rng(900 + i), (M, H), 1.0)
            dw = {n: dev(w[n]) for n in NAMES}
            mw = mtpx.moe_weights_from(dw, H, E, K, F, gs)
            out = (empty_bf16(M, H), torch.zeros(M, K, dtype=torch.int32, device="cuda"),
                   torch.zeros(M, K, dtype=torch.float32, device="cuda"),
                   torch.zeros(M, E, dtype=torch.float32, device="cuda"))
            c.moe_forward(mw, dev(x), *out)
            runs.append((w, x, E, M, out, dw))
        c.synchronize()
        for w, x, E, M, (y, idx, wt, lg), _ in runs:
            ref = O.moe_block(w, x, H, E, K, F, gs)
            assert np.array_equal(host(lg).view(np.uint32), ref["logits"].view(np.uint32))
            assert np.array_equal(host(idx), ref["idx"])
            assert np.array_equal(host(wt).view(np.uint32), ref["w"].view(np.uint32))
            assert np.array_equal(host(y), ref["y"])
    finally:
        c.close()


@pytest.mark.parametrize("H,E,K,F,gs,M", [(4096, 12, 4, 256, 64, 8), (1024, 16, 4, 320, 32, 5),
                                          (512, 8, 2, 1024, 32, 3)])
def test_moe_other_depths_bit_exact(ctx, H, E, K, F, gs, M):
    # H 4096 at M 8 leaves no LDS for a prefetch ring in gate|up; F 1024 fills the down staging
    print("case moe shape", H, E, K, F, gs, M, flush=True)
    w = make_moe(H + F + M, H, E, K, F, gs)
    run_case(ctx, w, H, E, K, F, gs, M, 31 + M, packed=True)
