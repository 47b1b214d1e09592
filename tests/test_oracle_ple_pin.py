"""Pins of the PLE n-gram block's oracle (oracle/mtpx_oracle.c o_ngram_row_ids,
o_ple_gate, o_ple_conv; oracle.ple_forward), on the CPU.

What fixes each piece:
  * head vocabularies: the design note's row total (docs/ngram-cache-design.md:84-89:
    16 heads, 320,001,446 rows) and shard geometry (:17-21: 128 shards x 2,500,012 rows)
    follow from "consecutive primes above ngram_vocab_size_base" with base 20,000,000;
  * the hash: closed forms with unit multipliers (each shifted copy on its own), XOR
    against ADD, the eos barrier, the non-negativity bound of :71-79 at its extreme;
  * the gate: float64 arithmetic of the same chain within bf16 rounding, plus the
    closed form of a zero key (dot 0 -> g 0 -> sigmoid 0.5);
  * the conv: single-tap kernels give gated + silu(one input row) exactly, which fixes
    the dilation, the tap order and the carried-row indexing; random taps against float64;
  * the block: a window split in two with the state carried gives the same bits.
The eos-barrier extent and the head order are the note's prose restated: the fork's
hash tests (Qwen4ExpNGramHashTests) are not in the tree, so the ids themselves are
parity unpinned against reference bits.
"""
import numpy as np
import pytest

from oracle import oracle as O

EOS = 248044


def test_head_vocabularies_match_the_design_note():
    v = O.primes_above(20_000_000, 16)
    assert sum(v) == 320_001_446
    assert -(-sum(v) // 128) == 2_500_012
    assert all(b > a for a, b in zip(v, v[1:]))


def _ids(hist, mult, vocab, offs, ctx=2, n=3, hpn=2, rows=None):
    rows = int(sum(vocab)) if rows is None else rows
    return O.ngram_row_ids(np.asarray(hist, np.int32), ctx, n, hpn, mult, vocab, offs, rows, EOS)


VOCAB = np.array(O.primes_above(1000, 4), np.int64)
OFFS = np.concatenate([[0], np.cumsum(VOCAB)[:-1]]).astype(np.int64)


def test_hash_unit_multipliers_select_each_shifted_copy():
    hist = [11, 222, 3333, 44444, 5555, 66]
    # copy 0 alone: the position's own token
    r = _ids(hist, [1, 0, 0], VOCAB, OFFS)
    for i, tok in enumerate(hist[2:]):
        assert list(r[i]) == [tok % VOCAB[h] + OFFS[h] for h in range(4)]
    # copy 1 alone: the previous token, for both widths
    r = _ids(hist, [0, 1, 0], VOCAB, OFFS)
    for i in range(4):
        assert list(r[i]) == [hist[i + 1] % VOCAB[h] + OFFS[h] for h in range(4)]
    # copy 2 alone: absent from width 2 (mix 0), two back for width 3
    r = _ids(hist, [0, 0, 1], VOCAB, OFFS)
    for i in range(4):
        assert list(r[i][:2]) == [OFFS[0], OFFS[1]]
        assert list(r[i][2:]) == [hist[i] % VOCAB[h] + OFFS[h] for h in (2, 3)]


def test_hash_mixes_by_xor():
    # equal copies with equal multipliers cancel under XOR (ADD would give 2t)
    hist = [7, 7, 7, 9, 9]
    r = _ids(hist, [5, 5, 0], VOCAB, OFFS)
    assert list(r[0][:2]) == [OFFS[0], OFFS[1]]  # position 2: copies 7, 7
    assert list(r[1][:2]) == [(9 * 5 ^ 7 * 5) % VOCAB[0] + OFFS[0], (9 * 5 ^ 7 * 5) % VOCAB[1] + OFFS[1]]
    assert list(r[2][:2]) == [OFFS[0], OFFS[1]]  # position 4: copies 9, 9


def test_hash_never_crosses_an_eos():
    # width 3 at a token right after an eos: copy 2 would cross it and reads eos instead
    a = _ids([100, 200, EOS, 300], [3, 5, 7], VOCAB, OFFS)
    b = _ids([999, 888, EOS, 300], [3, 5, 7], VOCAB, OFFS)
    assert np.array_equal(a[1], b[1])
    mix3 = (300 * 3) ^ (EOS * 5) ^ (EOS * 7)
    assert list(a[1][2:]) == [mix3 % VOCAB[h] + OFFS[h] for h in (2, 3)]
    # the eos token itself still sees the two tokens before it
    mix3e = (EOS * 3) ^ (200 * 5) ^ (100 * 7)
    assert list(a[0][2:]) == [mix3e % VOCAB[h] + OFFS[h] for h in (2, 3)]


def test_hash_stays_non_negative_at_the_multiplier_bound():
    V = 248320
    bound = (2 ** 63 - 1) // V // 2
    m = bound - 1 if (bound - 1) % 2 else bound - 2  # the largest odd multiplier below the bound
    vocab = np.array(O.primes_above(20_000_000, 4), np.int64)
    offs = np.concatenate([[0], np.cumsum(vocab)[:-1]]).astype(np.int64)
    hist = [V - 1, V - 2, V - 1, V - 3, 0, V - 1]
    r = _ids(hist, [m, m - 2, m - 4], vocab, offs)
    assert (r >= 0).all()
    for h in range(4):
        assert ((r[:, h] >= offs[h]) & (r[:, h] < offs[h] + vocab[h])).all()
    # python integers as the independent 64-bit check of one id
    mix = ((V - 1) * m) ^ ((V - 2) * (m - 2)) ^ ((V - 1) * (m - 4))
    assert mix < 2 ** 63 and r[0, 2] == mix % vocab[2] + offs[2]


def test_hash_out_of_table_ids_are_flagged():
    r = _ids([1, 2, 3], [1, 0, 0], VOCAB, OFFS, rows=int(OFFS[2]))  # heads 2 and 3 fall outside
    assert list(r[0][2:]) == [-1, -1] and (r[0][:2] >= 0).all()


def _bf(r, shape, sigma=1.0):
    return O.f32_to_bf16((r.standard_normal(shape) * sigma).astype(np.float32))


def _f(x):
    return O.bf16_to_f32(x).astype(np.float64)


@pytest.mark.parametrize("H", [256, 2560])
def test_ple_gate_against_float64(H):
    r = np.random.default_rng(H)
    for trial in range(4):
        key, stream, value = _bf(r, H, 2.0), _bf(r, H), _bf(r, H)
        ks, qs, cs = (O.f32_to_bf16((1 + 0.2 * r.standard_normal(H)).astype(np.float32)) for _ in range(3))
        gated, normed, dot = O.ple_gate(key, stream, value, ks, qs, cs, 1e-6)
        k, q = _f(key), _f(stream)
        kn = k / np.sqrt((k * k).mean() + 1e-6) * _f(ks)
        qn = q / np.sqrt((q * q).mean() + 1e-6) * _f(qs)
        p = kn * qn
        # bf16 products and a bf16 row sum: within a few bf16 steps of the magnitude summed
        assert abs(dot - p.sum()) <= 2 ** -6 * np.abs(p).sum() + 1e-3
        g = dot / float(O.bf16_to_f32(O.f32_to_bf16(np.array([np.sqrt(H)], np.float32)))[0])
        g = np.sign(g) * np.sqrt(max(abs(g), 1e-6))
        sgm = 1 / (1 + np.exp(-g))
        want = sgm * _f(value)
        assert np.allclose(_f(gated), want, rtol=2 ** -6, atol=1e-6)
        v = _f(gated)
        want_n = v / np.sqrt((v * v).mean() + 1e-6) * _f(cs)
        assert np.allclose(_f(normed), want_n, rtol=2 ** -6, atol=2 ** -6 * np.abs(want_n).max())


def test_ple_gate_sign_follows_the_dot():
    # a negated key negates every product and the bf16 sum exactly; the gate then uses sigmoid(-g)
    r = np.random.default_rng(4)
    H = 2560
    key, stream, value = _bf(r, H, 2.0), _bf(r, H), _bf(r, H)
    ones = O.f32_to_bf16(np.ones(H, np.float32))
    g1, _, d1 = O.ple_gate(key, stream, value, ones, ones, ones, 1e-6)
    g2, _, d2 = O.ple_gate(key ^ np.uint16(0x8000), stream, value, ones, ones, ones, 1e-6)
    assert d1 != 0.0 and d2 == -d1
    s1 = 1 / (1 + np.exp(-np.sign(d1) * np.sqrt(abs(d1) / np.sqrt(H))))
    assert np.allclose(_f(g1), s1 * _f(value), rtol=2 ** -6, atol=1e-6)
    assert np.allclose(_f(g2), (1 - s1) * _f(value), rtol=2 ** -6, atol=1e-6)


def test_ple_gate_zero_key_closed_form():
    r = np.random.default_rng(3)
    H = 512
    key = np.zeros(H, np.uint16)
    stream, value = _bf(r, H), _bf(r, H)
    ones = O.f32_to_bf16(np.ones(H, np.float32))
    gated, _, dot = O.ple_gate(key, stream, value, ones, ones, ones, 1e-6)
    assert dot == 0.0
    assert np.array_equal(gated, O.f32_to_bf16(O.bf16_to_f32(value) * np.float32(0.5)))


def test_ple_conv_single_taps_fix_the_indexing():
    r = np.random.default_rng(5)
    S, W, kc, dil = 3, 64, 4, 3
    nb = (kc - 1) * dil
    full = _bf(r, (nb + S, W))
    gated = _bf(r, (S, W))
    for j in range(kc):
        cw = np.zeros((W, kc), np.uint16)
        cw[:, j] = O.f32_to_bf16(np.ones(W, np.float32))
        out = O.ple_conv(full, cw, gated, dil)
        x = full[np.arange(S) + j * dil]
        want = O.f32_to_bf16(O.bf16_to_f32(gated) + O.bf16_to_f32(O.silu_rows(x)))
        assert np.array_equal(out, want), j


def test_ple_conv_random_taps_against_float64():
    r = np.random.default_rng(6)
    S, W, kc, dil = 5, 128, 4, 3
    full = _bf(r, ((kc - 1) * dil + S, W))
    gated = _bf(r, (S, W))
    cw = _bf(r, (W, kc), 0.3)
    out = O.ple_conv(full, cw, gated, dil)
    acc = np.stack([sum(_f(full[t + j * dil]) * _f(cw[:, j]) for j in range(kc)) for t in range(S)])
    want = _f(gated) + acc / (1 + np.exp(-acc))
    assert np.allclose(_f(out), want, rtol=2 ** -6, atol=2 ** -7)


def small_ple(r, H=256, hc=2, E=256, n=3, hpn=2, kc=4, gs=32, base=500):
    nh = (n - 1) * hpn
    rd = E // nh
    vocab = np.array(O.primes_above(base, nh), np.int64)
    offs = np.concatenate([[0], np.cumsum(vocab)[:-1]]).astype(np.int64)
    rows = int(vocab.sum())
    W = hc * H
    table = O.affine_quantize(_bf(r, (rows, rd), 0.5), 32)
    w = dict(key_proj=O.affine_quantize(_bf(r, (W, E), 0.05), gs), value_proj=O.affine_quantize(_bf(r, (H, E), 0.05), gs),
             norm_key=O.f32_to_bf16((1 + 0.1 * r.standard_normal(W)).astype(np.float32)),
             norm_query=O.f32_to_bf16((1 + 0.1 * r.standard_normal(W)).astype(np.float32)),
             norm_conv=O.f32_to_bf16((1 + 0.1 * r.standard_normal(W)).astype(np.float32)),
             conv_w=_bf(r, (W, kc), 0.3), table=table, mult=np.array([3, 1000003, 7919], np.int64), vocab=vocab,
             offs=offs)
    cfg = dict(hidden=H, hc=hc, embed_dim=E, ngram_size=n, heads_per_ngram=hpn, conv_kernel=kc, group_size=gs,
               row_group_size=32, eos=EOS, eps=1e-6)
    return w, cfg


def test_ple_window_split_gives_the_same_bits():
    r = np.random.default_rng(9)
    w, cfg = small_ple(r)
    W, nb = cfg["hc"] * cfg["hidden"], 3 * 3
    conv = _bf(r, (nb, W))
    ctx = np.array([17, EOS], np.int32)
    ids = np.array([5, 900, EOS, 33, 4], np.int32)
    stream = _bf(r, (5, W))
    whole = O.ple_forward(w, cfg, stream, ids, conv, ctx)
    first = O.ple_forward(w, cfg, stream[:2], ids[:2], conv, ctx)
    conv2, ctx2 = O.ple_advance(first, 2, nb, 2)
    second = O.ple_forward(w, cfg, stream[2:], ids[2:], conv2, ctx2)
    assert np.array_equal(np.concatenate([first["out"], second["out"]]), whole["out"])
    assert np.array_equal(np.concatenate([first["row_ids"], second["row_ids"]]), whole["row_ids"])
    # the block's embedding is the table's rows in head order
    assert (whole["row_ids"] >= 0).all()
    emb = whole["embedded"].reshape(5, 4, -1)
    assert np.array_equal(emb[3, 1], O.embed_rows(*w["table"], 32, whole["row_ids"][3, 1:2])[0])
