"""Pins the CPU oracle (oracle/qp_oracle.py) to facts that do not come from its own formulas.

| oracle function          | pinned by                                                                                  |
|--------------------------|--------------------------------------------------------------------------------------------|
| f32_to_bf16_bits         | IEEE known answers (ties to even, inf, NaN) and torch's independent bf16 cast               |
| int4/k8v4 views, cells   | literal byte layouts of the reference tests (tests/test_k8v4_kv.py:16-46, spec 264/392)     |
| unpack_int4 / unpack_i8  | hand-computed cells (nibble order, zero point in the word's low bits, masked scale)         |
| dequant_f64, attention   | pure-Python brute force on a tiny case; causality; constant-V closed form                   |
| decode_partials + merge  | fp64 attention within 1e-2 (reference bound, tests/test_int4_kv.py:190) and 0.5%;           |
|                          | single-tile = textbook softmax; segment-count invariance; constant V; planted mistakes     |
| merge_partials           | two-segment closed form (LSE algebra)                                                       |
| segment_lse, merge_lse   | scipy's logsumexp of the scores (natural log), a pure-Python loop, empty segments -> -inf   |
| value_probabilities      | planted mistake: the zero-point sum taken on the unrounded P * s_v fails fp64 where the     |
|                          | value codes equal their zero points on all but two keys                                    |
| max_row_relerr           | hand-computed rows                                                                          |
| quantize_int4 (_fma32)   | rows where FMA and mul-then-add round differently: the oracle takes the FMA code (assumed,  |
|                          | parity unpinned against the reference's Triton store)                                       |
| quantize_int4/int8/store | reference error bounds (tests/test_k8v4_kv.py:147-156), hand-built rows, slot -1 skipped,   |
|                          | the 1e-6 scale floors on all-zero and constant rows (known answers from k8v4_ops.py:35,52) |
| round_half_away          | known answers incl. fp32 `x + 0.5` rounding                                                 |
| rht                      | R R^T = hs I, Sylvester entries (-1)^popcount(i & j), pure-Python hash of the signs          |
| prefill_dequant_attend   | fp64 attention within 1e-2                                                                  |
| quantize_query_i8        | hand rows (half to even, the 1e-20 floor), the reconstruction bound, torch running the       |
|                          | reference's own lines (int4_prefill.py:181-189) bit for bit                                 |
| i8_scores                | term-by-term brute force of the integer dots and the two fp32 products                     |
| prefill_i8_emulated      | fp64 within 0.2 %; four planted mistakes (hi part alone, no key / value zero point, the     |
|                          | query sum weighted 256) each fail it                                                        |
"""
import numpy as np
import pytest

from oracle import qp_oracle as O


# ------------------------------------------------------------------------------------------------------ bf16

def test_bf16_known_answers():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)
    cases = {
        1.0: 0x3F80,
        float(one + ulp / 2): 0x3F80,             # tie -> even (0x3F80)
        float(one + ulp + ulp / 2): 0x3F82,       # tie -> even (0x3F82)
        float(one + ulp / 2 + np.float32(2.0 ** -20)): 0x3F81,
        -2.0: 0xC000,
        np.inf: 0x7F80,
        -0.0: 0x8000,
        3.3895313892515355e38: 0x7F7F,            # the largest finite bf16
        3.4e38: 0x7F80,                           # past the halfway point to 2^128: inf
    }
    for x, want in cases.items():
        assert int(O.f32_to_bf16_bits(np.float32(x))) == want, x
    assert np.isnan(O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.float32(np.nan))))


def test_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1e3
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (O.f32_to_bf16_bits(x) == want).all()


# ----------------------------------------------------------------------------------------------- cells / views

def test_cell_sizes_match_reference_literals():
    assert O.k8v4_cell_bytes(256, 256) == 392
    assert O.k8v4_cell_bytes(128, 64) == 168
    assert O.int4_cell_bytes(256) == 264


@pytest.mark.parametrize("layout", ["hnd", "nhd"])
def test_k8v4_views_cover_the_cell_without_overlap(layout):
    """tests/test_k8v4_kv.py:21-41 restated on the numpy views."""
    nb, nkv, bs, hs = 3, 2, 4, 16
    kv = O.new_cache(nb, nkv, bs, O.k8v4_cell_bytes(hs), layout)
    v = O.k8v4_views(kv, hs)
    assert v.key.shape == (nb, bs, nkv, hs) and v.key.dtype == np.int8
    assert v.value.shape == (nb, bs, nkv, hs // 2) and v.value.dtype == np.uint8
    assert v.key_word.shape == v.value_word.shape == (nb, bs, nkv)
    v.key[...] = 1
    v.key_word[...] = 0x02020202
    v.value[...] = 3
    v.value_word[...] = 0x04040404
    want = np.array([1] * hs + [2] * 4 + [3] * (hs // 2) + [4] * 4, np.uint8)
    assert (kv == want).all()
    v.key_word[1, 2, 1] = np.float32(7.0).view(np.uint32)
    assert kv[1, 1, 2, hs:hs + 4].copy().view(np.float32)[0] == 7.0


def test_k8v4_views_reject_another_cell_size():
    with pytest.raises(ValueError, match="expected 392"):
        O.k8v4_views(np.zeros((1, 4, 16, 264), np.uint8), 256)


def test_int4_views_layout():
    """[K nibbles hs/2 | K word | V nibbles hs/2 | V word] per (block, head, slot) cell (tests/test_int4_kv.py:95-103)."""
    nb, nkv, bs, hs = 2, 3, 4, 8
    kv = O.new_cache(nb, nkv, bs, O.int4_cell_bytes(hs))
    v = O.int4_views(kv, hs)
    v.key[...] = 0x11
    v.key_word[...] = 0x22222222
    v.value[...] = 0x33
    v.value_word[...] = 0x44444444
    want = np.array([0x11] * 4 + [0x22] * 4 + [0x33] * 4 + [0x44] * 4, np.uint8)
    assert (kv == want).all()
    v.value[1, 3, 2, 0] = 0xAB                       # (block, slot, head) of a view = (block, head, slot) of the cache
    assert kv[1, 2, 3, hs // 2 + 4] == 0xAB


# ------------------------------------------------------------------------------------------------------ unpack

def _word(scale: float, zp: int) -> np.uint32:
    return np.uint32((int(np.float32(scale).view(np.uint32)) & 0xFFFFFFF0) | zp)


def test_unpack_int4_hand_computed():
    w = _word(0.05, 7)
    s = float(np.uint32(int(w) & 0xFFFFFFF0).view(np.float32))
    codes = np.array([[0x9A, 0x07, 0xF0]], np.uint8)     # channels: 10, 9, 7, 0, 0, 15
    got = O.bf16_bits_to_f32(O.unpack_int4(codes, np.array([w])))
    want = np.array([3, 2, 0, -7, -7, 8], np.float64) * s
    assert np.allclose(got[0], want, rtol=2 ** -8, atol=0)
    assert got[0, 2] == 0.0                              # nibble == zero point is exactly zero
    # the scale is the word with its low 4 bits cleared: a word whose low bits are 0xF decodes to the same scale
    assert (O.unpack_int4(codes, np.array([np.uint32(int(w) | 0xF)]))
            != O.unpack_int4(codes, np.array([w]))).any()          # zp changed 7 -> 15 ...
    z15 = O.bf16_bits_to_f32(O.unpack_int4(codes, np.array([np.uint32(int(w) | 0xF)])))[0]
    assert np.allclose(z15, (np.array([10, 9, 7, 0, 0, 15]) - 15) * s, rtol=2 ** -8)   # ... scale unchanged


def test_unpack_int4_single_rounding():
    """fp32 product then one RNE to bf16: equal to torch doing the same steps on the hand-decoded fields."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, (64, 128), dtype=np.uint8)
    words = np.array([_word(s, z) for s, z in zip(rng.lognormal(-3, 0.5, 64), rng.integers(0, 16, 64))])
    u = np.empty((64, 256), np.float32)
    u[:, 0::2], u[:, 1::2] = codes & 0xF, codes >> 4
    zp = torch.tensor((words & 0xF).astype(np.float32))
    sc = torch.tensor((words & np.uint32(0xFFFFFFF0)).view(np.float32))
    want = ((torch.from_numpy(u) - zp[:, None]) * sc[:, None]).to(torch.bfloat16).view(torch.int16).numpy()
    assert (O.unpack_int4(codes, words).view(np.int16) == want).all()


def test_unpack_i8_hand_computed():
    s = np.float32(0.0123)
    codes = np.array([[-127, -1, 0, 5, 127]], np.int8)
    got = O.bf16_bits_to_f32(O.unpack_i8(codes, np.array([s]).view(np.uint32)))[0]
    assert np.allclose(got, codes[0] * float(s), rtol=2 ** -8)
    assert got[2] == 0.0 and got[0] == -got[4]


def test_unpack_segment_follows_the_block_table():
    nb, nkv, bs, hs = 6, 2, 4, 8
    kv = O.new_cache(nb, nkv, bs, O.int4_cell_bytes(hs))
    v = O.int4_views(kv, hs)
    for b in range(nb):
        v.key[b] = b * 16 + 1                            # nibbles (1, b)
        v.key_word[b] = _word(1.0, 0)
    row = np.array([5, 2, 0], np.int32)
    out = O.bf16_bits_to_f32(O.unpack_segment(v, row, 3, 6, "key"))   # positions 3..8 -> blocks 5, 2, 2, 2, 2, 0
    assert out.shape == (6, nkv, hs)
    assert list(out[:, 0, 1]) == [5, 2, 2, 2, 2, 0]
    assert (out[:, :, 0::2] == 1).all()


# ---------------------------------------------------------------------------------------------- attention f64

def _tiny_cache(rng, n, nkv, hs, bs, fmt="int4"):
    nb = -(-n // bs) + 2
    if fmt == "int4":
        kv = O.new_cache(nb, nkv, bs, O.int4_cell_bytes(hs))
        v = O.int4_views(kv, hs)
        v.key[...] = rng.integers(0, 256, v.key.shape, dtype=np.uint8)
        v.key_word[...] = np.array([_word(s, z) for s, z in zip(rng.lognormal(-3, .5, v.key_word.size),
                                                                rng.integers(6, 10, v.key_word.size))]
                                   ).reshape(v.key_word.shape)
    else:
        kv = O.new_cache(nb, nkv, bs, O.k8v4_cell_bytes(hs))
        v = O.k8v4_views(kv, hs)
        v.key[...] = rng.integers(-127, 128, v.key.shape, dtype=np.int8)
        v.key_word[...] = rng.lognormal(-4, .5, v.key_word.shape).astype(np.float32).view(np.uint32)
    v.value[...] = rng.integers(0, 256, v.value.shape, dtype=np.uint8)
    v.value_word[...] = np.array([_word(s, z) for s, z in zip(rng.lognormal(-3, .5, v.value_word.size),
                                                              rng.integers(6, 10, v.value_word.size))]
                                 ).reshape(v.value_word.shape)
    row = rng.permutation(nb)[: -(-n // bs)].astype(np.int32)
    return v, row


def test_attention_f64_brute_force():
    rng = np.random.default_rng(2)
    T, NQ, nkv, hs, n = 2, 4, 2, 4, 5
    q = rng.standard_normal((T, NQ, hs))
    K = rng.standard_normal((n, nkv, hs))
    V = rng.standard_normal((n, nkv, hs))
    got = O.attention_f64(q, K, V, n, 0.7)
    import math
    for t in range(T):
        for h in range(NQ):
            kh = h // (NQ // nkv)
            vis = n - T + t + 1
            sc = [0.7 * sum(q[t, h, c] * K[j, kh, c] for c in range(hs)) for j in range(vis)]
            mx = max(sc)
            e = [math.exp(s - mx) for s in sc]
            for c in range(hs):
                want = sum(e[j] * V[j, kh, c] for j in range(vis)) / sum(e)
                assert abs(got[t, h, c] - want) < 1e-12


def test_dequant_f64_matches_hand_formula():
    rng = np.random.default_rng(3)
    v, row = _tiny_cache(rng, 40, 2, 8, 16)
    K, V = O.dequant_f64(v, row, 40)
    b, s = row[33 // 16], 33 % 16
    byte = int(v.key[b, s, 1, 3])
    w = int(v.key_word[b, s, 1])
    scale = float(np.uint32(w & 0xFFFFFFF0).view(np.float32))
    assert K[33, 1, 6] == ((byte & 0xF) - (w & 0xF)) * scale
    assert K[33, 1, 7] == ((byte >> 4) - (w & 0xF)) * scale


# ------------------------------------------------------------------------------- exact kernel emulation + merge

@pytest.mark.parametrize("fmt", ["int4", "int8"])
@pytest.mark.parametrize("T", [1, 2, 4])
def test_emulation_matches_fp64(fmt, T):
    rng = np.random.default_rng(10 + T)
    n, nq, nkv, hs = 700, 6, 2, 32
    v, row = _tiny_cache(rng, n, nkv, hs, 16, fmt)
    q = O.round_bf16(rng.standard_normal((T, nq, hs)).astype(np.float32))
    scale = hs ** -0.5
    K, V = O.dequant_f64(v, row, n)
    ref = O.attention_f64(q, K, V, n, scale)
    for S in (1, 3, 8):
        got = O.decode_emulated(q, v, row, n, scale, num_segments=S)
        e = O.relerr(got, ref)
        assert e < 5e-3, (S, e)


def test_emulation_single_tile_is_textbook_softmax():
    rng = np.random.default_rng(4)
    n, hs = 50, 16
    v, row = _tiny_cache(rng, n, 1, hs, 16)
    q = O.round_bf16(rng.standard_normal((1, 3, hs)).astype(np.float32))
    K, V = O.dequant_f64(v, row, n)
    s = np.einsum("hc,nc->hn", q[0].astype(np.float64), K[:, 0]) * 0.25
    p = np.exp(s - s.max(1, keepdims=True))
    want = (p / p.sum(1, keepdims=True)) @ V[:, 0]
    got = O.decode_emulated(q, v, row, n, 0.25)[0]
    assert O.relerr(got, want) < 3e-3


def test_emulation_segment_count_invariance():
    rng = np.random.default_rng(5)
    n = 1000
    v, row = _tiny_cache(rng, n, 2, 32, 16)
    q = O.round_bf16(rng.standard_normal((2, 4, 32)).astype(np.float32))
    base = O.merge_partials(*O.decode_partials(q, v, row, n, 0.2, 1))
    for S in (2, 5, 16, 40):
        got = O.merge_partials(*O.decode_partials(q, v, row, n, 0.2, S))
        assert O.relerr(got, base) < 2e-3, S


def test_emulation_constant_value_closed_form():
    """Every value nibble c with zero point z and scale s: the output is (c - z) * s for every row."""
    rng = np.random.default_rng(6)
    n, hs = 300, 16
    v, row = _tiny_cache(rng, n, 1, hs, 16)
    v.value[...] = 0x33                                  # c = 3 in both nibbles
    w = _word(0.125, 9)
    v.value_word[...] = w
    q = O.round_bf16(rng.standard_normal((2, 2, hs)).astype(np.float32))
    got = O.decode_emulated(q, v, row, n, 0.3, num_segments=4)
    assert np.allclose(got, (3 - 9) * 0.125, rtol=4e-3)


def test_emulation_is_causal():
    rng = np.random.default_rng(7)
    n, hs = 200, 16
    v, row = _tiny_cache(rng, n, 1, hs, 16)
    q = O.round_bf16(rng.standard_normal((2, 1, hs)).astype(np.float32))
    a = O.decode_emulated(q, v, row, n, 0.3, num_segments=3)
    v.value[row[(n - 1) // 16], (n - 1) % 16] ^= 0xFF        # the newest key: visible to the second token only
    b = O.decode_emulated(q, v, row, n, 0.3, num_segments=3)
    assert (a[0] == b[0]).all() and not (a[1] == b[1]).all()


def test_merge_two_segments_closed_form():
    rng = np.random.default_rng(8)
    s = rng.standard_normal(20) * 3
    x = rng.standard_normal((20, 5))
    full = (np.exp(s - s.max()) @ x) / np.exp(s - s.max()).sum()
    parts = []
    for lo, hi in ((0, 7), (7, 20)):
        m = s[lo:hi].max()
        p = np.exp2((s[lo:hi] - m) * O.LOG2E)   # base-2 units, as the kernels keep m
        parts.append(((p @ x[lo:hi]).astype(np.float32), np.float32(m * O.LOG2E), np.float32(p.sum())))
    acc = np.stack([p[0] for p in parts])[None]
    m = np.array([p[1] for p in parts], np.float32)[None]
    l_ = np.array([p[2] for p in parts], np.float32)[None]
    got = O.merge_partials(acc, m, l_)[0]
    assert np.allclose(got, full, rtol=1e-5, atol=1e-6)


# planted mistakes: each variant of the emulation must fail the fp64 check that the real one passes
def _planted(monkeypatch, kind):
    real_parts = O.int4_word_parts
    if kind == "drop-zero-point":
        monkeypatch.setattr(O, "int4_word_parts", lambda w: (np.zeros_like(real_parts(w)[0]), real_parts(w)[1]))
    elif kind == "swap-nibbles":
        real_gather = O.gather

        def gather(views, row, pos):
            kc, kw, vc, vw = real_gather(views, row, pos)
            sw = lambda c: ((c & 0xF) << 4) | (c >> 4)
            return (sw(kc) if views.key_format == "int4" else kc), kw, sw(vc), vw
        monkeypatch.setattr(O, "gather", gather)
    elif kind == "unmasked-scale":
        monkeypatch.setattr(O, "int4_word_parts", lambda w: (real_parts(w)[0], np.asarray(w, np.uint32).view(
            np.float32) * np.float32(1.5)))


@pytest.mark.parametrize("kind", ["drop-zero-point", "swap-nibbles", "unmasked-scale"])
def test_planted_mistakes_fail_the_fp64_check(monkeypatch, kind):
    rng = np.random.default_rng(9)
    n, hs = 400, 32
    v, row = _tiny_cache(rng, n, 2, hs, 16)
    q = O.round_bf16(rng.standard_normal((2, 4, hs)).astype(np.float32))
    K, V = O.dequant_f64(v, row, n)
    ref = O.attention_f64(q, K, V, n, 0.2)
    assert O.relerr(O.decode_emulated(q, v, row, n, 0.2, 2), ref) < 5e-3
    _planted(monkeypatch, kind)
    assert O.relerr(O.decode_emulated(q, v, row, n, 0.2, 2), ref) > 2e-2


# -------------------------------------------------------------------------------------------------- store

def test_round_half_away_known_answers():
    x = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997, 2.4999998, 7.0], np.float32)
    want = np.array([1, -1, 2, 3, -3, 1, -1, 2, 7], np.float32)   # 0.49999997 + 0.5 rounds to 1.0 in fp32
    assert (O.round_half_away(x) == want).all()


def test_quantize_int4_hand_row():
    v = np.arange(16, dtype=np.float32) - 1.0          # min -1, max 14: scale 1, zero point 1, codes 0..15
    codes, word = O.quantize_int4(v[None])
    assert int(word[0]) & 0xF == 1
    assert np.uint32(int(word[0]) & 0xFFFFFFF0).view(np.float32) == np.float32(1.0)
    u = np.empty(16, np.int64)
    u[0::2], u[1::2] = codes[0] & 0xF, codes[0] >> 4
    assert (u == np.arange(16)).all()


def test_quantize_int8_hand_row():
    k = np.array([[-2.54, 0.0, 1.27, 2.54]], np.float32)
    q, w = O.quantize_int8(k)
    s = w.view(np.float32)[0]
    assert s == np.float32(np.float32(2.54) / np.float32(127.0))
    assert list(q[0]) == [-127, 0, 64, 127]            # 1.27 / 0.02 = 63.5 -> half away from zero -> 64


# Rows with no spread, where the reference's max(., 1e-6) floors set the scale (k8v4_ops.py:35,52): fp32(1e-6) has
# the bits 0x358637BD, which the int4 word keeps with its low four bits replaced by the zero point (:58). Each row:
# (value of every channel, int4 code bytes, int4 word, int8 codes, int8 scale bits), derived by hand from the steps
#   zero row:   scale 1e-6; zp = round(-0 / 1e-6) = 0 (-0.0 >= 0 takes x + 0.5); codes round(0 * 1e6 + 0) = 0;
#               int8: scale max(0 / 127, 1e-6) = 1e-6, codes 0;
#   row 0.5:    scale 1e-6; zp = round(-5e5) -> clamp 0; codes round(5e5) -> clamp 15 (bytes 0xFF);
#               int8: scale 0.5 / 127 (above the floor), codes 127;
#   row -0.5:   zp = round(5e5) -> clamp 15; codes round(-5e5 + 15) -> clamp 0; int8 codes -127;
#   row 1e-5:   scale 1e-6; zp = round(-10.01) -> clamp 0; codes round(bf16(1e-5) * 1e6) = round(10.01) = 10 (bytes
#               0xAA); int8: scale max(1e-5 / 127, 1e-6) = 1e-6, codes round(10.01) = 10.
FLOOR = 0x358637BD
DEGENERATE_ROWS = [(0.0, 0x00, FLOOR & ~0xF, 0, FLOOR),
                   (0.5, 0xFF, FLOOR & ~0xF, 127, None),
                   (-0.5, 0x00, (FLOOR & ~0xF) | 15, -127, None),
                   (1.001358e-05, 0xAA, FLOOR & ~0xF, 10, FLOOR)]


def degenerate_rows(hs):
    """[len(DEGENERATE_ROWS), hs] fp32 rows of one repeated bf16 value each."""
    return np.array([np.full(hs, O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.float32(v)))) for v, *_ in
                     DEGENERATE_ROWS], np.float32)


def test_store_scale_floor_on_rows_without_spread():
    """The 1e-6 floors of both halves, on all-zero and constant rows (known answers above): a store without them
    divides by a zero scale and writes a zero scale word."""
    x = degenerate_rows(16)
    codes, words = O.quantize_int4(x)
    for i, (v, byte, word, k8, k8_bits) in enumerate(DEGENERATE_ROWS):
        assert (codes[i] == byte).all(), v
        assert int(words[i]) == word, (v, hex(int(words[i])))
    q, bits = O.quantize_int8(x)
    for i, (v, byte, word, k8, k8_bits) in enumerate(DEGENERATE_ROWS):
        assert (q[i] == k8).all(), v
        want = k8_bits if k8_bits is not None else int(np.float32(abs(np.float32(v)) / np.float32(127.0)).view(np.uint32))
        assert int(bits[i]) == want, (v, hex(int(bits[i])))
    # a row whose spread is below the floor: 0 and bf16(1e-6) = 9.98e-7 give codes 0 and round(0.998) = 1
    tiny = np.zeros((1, 16), np.float32)
    tiny[0, 15] = O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.float32(1e-6)))
    c, w = O.quantize_int4(tiny)
    assert int(w[0]) == FLOOR & ~0xF and list(c[0]) == [0] * 7 + [0x10]


def test_store_error_bounds_and_skipped_slots():
    """tests/test_k8v4_kv.py:140-156: int8 keys < 2 % error, int4 values 5-20 %, slot -1 leaves the cache alone."""
    rng = np.random.default_rng(11)
    n, nkv, hs = 512, 2, 64
    kv = O.new_cache(-(-n // 16), nkv, 16, O.k8v4_cell_bytes(hs))
    v = O.k8v4_views(kv, hs)
    k = rng.standard_normal((n, nkv, hs)).astype(np.float32)
    x = rng.standard_normal((n, nkv, hs)).astype(np.float32)
    O.store(v, k, x, np.arange(n))
    K, V = O.dequant_f64(v, np.arange(kv.shape[0]), n)
    assert O.relerr(K, k) < 0.02
    assert 0.05 < O.relerr(V, x) < 0.2
    before = kv.copy()
    O.store(v, k[:8], x[:8], np.full(8, -1))
    assert (kv == before).all()


# ---------------------------------------------------------------------------------------------------- RHT

def _lowbias32(c: int, seed: int = 0) -> int:
    x = (c + seed * 0x9E3779B9) & 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x


def test_rht_signs_pure_python_hash():
    for seed in (0, 3):
        want = [-1.0 if _lowbias32(c, seed) & 1 else 1.0 for c in range(256)]
        assert list(O.rht_signs(256, seed)) == want
    assert 64 < (O.rht_signs(256) < 0).sum() < 192


def test_rht_is_unnormalised_orthogonal():
    hs = 64
    H = O.sylvester(hs)
    i, j = np.meshgrid(np.arange(hs), np.arange(hs), indexing="ij")
    popc = np.vectorize(lambda v: bin(v).count("1"))(i & j)
    assert (H == (-1.0) ** popc).all()
    R = O.rht(np.eye(hs))                 # rows of I rotated: R^T
    assert np.allclose(R @ R.T, hs * np.eye(hs))
    x = np.random.default_rng(0).standard_normal((5, hs))
    assert np.allclose(O.rht(O.rht(x), inverse=True) / hs, x)
    y = O.rht(x)
    assert np.allclose((y * y).sum(1), hs * (x * x).sum(1))


# ------------------------------------------------------------------------------------------ CPU dequant path

@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_torch_unpack_equals_numpy_unpack(fmt):
    pytest.importorskip("torch")
    rng = np.random.default_rng(14)
    v, row = _tiny_cache(rng, 300, 2, 32, 16, fmt)
    kc, kw, vc, vw = O.gather(v, row, np.arange(300))
    want = O.unpack_i8(kc, kw) if fmt == "int8" else O.unpack_int4(kc, kw)
    assert (O.f32_to_bf16_bits(O.unpack_torch(kc, kw, fmt).numpy()) == want).all()
    assert (O.f32_to_bf16_bits(O.unpack_torch(vc, vw).numpy()) == O.unpack_int4(vc, vw)).all()


def test_dequant_then_attend_matches_fp64():
    pytest.importorskip("torch")
    rng = np.random.default_rng(13)
    n, hs = 3000, 32
    v, row = _tiny_cache(rng, n, 2, hs, 16)
    q = O.round_bf16(rng.standard_normal((64, 6, hs)).astype(np.float32))
    K, V = O.dequant_f64(v, row, n)
    ref = O.attention_f64(q, K, V, n, 0.2)
    got = O.prefill_dequant_attend(q, v, row, n, 0.2, segment=1024)
    assert O.relerr(got, ref) < 1e-2


# ----------------------------------------------------------------------------------------- log-sum-exp statistics

def _lse_loop(scores):
    import math
    mx = max(scores)
    return mx + math.log(sum(math.exp(x - mx) for x in scores))


def test_segment_and_merged_lse_closed_form():
    """(m, l) of a segment in log2 units, as the kernels keep them, give the natural-log LSE of its scores."""
    from scipy.special import logsumexp
    rng = np.random.default_rng(30)
    s = rng.standard_normal(37) * 4.0                          # natural-log scores of one row
    bounds = [(0, 10), (10, 10), (10, 37)]                       # the middle segment is empty
    ms, ls = [], []
    for lo, hi in bounds:
        if lo == hi:
            ms.append(-np.inf)
            ls.append(0.0)
            continue
        m = (s[lo:hi] * O.LOG2E).max()
        ms.append(m)
        ls.append(np.exp2(s[lo:hi] * O.LOG2E - m).sum())
    ms, ls = np.array(ms, np.float32), np.array(ls, np.float32)
    seg = O.segment_lse(ms, ls)
    for k, (lo, hi) in enumerate(bounds):
        if lo == hi:
            assert seg[k] == -np.inf
        else:
            assert abs(seg[k] - logsumexp(s[lo:hi])) < 2e-5
            assert abs(seg[k] - _lse_loop(list(s[lo:hi]))) < 2e-5
    assert abs(O.merge_lse(ms[None], ls[None])[0] - logsumexp(s)) < 2e-5
    assert O.merge_lse(np.full((1, 3), -np.inf, np.float32), np.zeros((1, 3), np.float32))[0] == -np.inf


def test_emulated_partials_give_the_fp64_lse():
    """The emulation's per-segment (m, l), folded, equal the fp64 logsumexp of scale * q . k over the visible keys."""
    from scipy.special import logsumexp
    rng = np.random.default_rng(31)
    n, nq, nkv, hs, T = 500, 4, 2, 32, 2
    for fmt in ("int4", "int8"):
        v, row = _tiny_cache(rng, n, nkv, hs, 16, fmt)
        q = O.round_bf16(rng.standard_normal((T, nq, hs)).astype(np.float32))
        _, m, l = O.decode_partials(q, v, row, n, 0.3, 5, tile=32)
        K, _ = O.dequant_f64(v, row, n)
        got = O.merge_lse(m, l)
        for t in range(T):
            for h in range(nq):
                vis = n - T + t + 1
                want = logsumexp(0.3 * (K[:vis, h // (nq // nkv)] @ q[t, h].astype(np.float64)))
                assert abs(got[t, h] - want) < 1e-4, (fmt, t, h)


def _dead_values(rng, v, row, n, live):
    """Value codes equal to their zero point (value 0) on every key but `live` random ones."""
    zp = (v.value_word & np.uint32(0xF)).astype(np.uint8)
    v.value[...] = zp[..., None] | (zp[..., None] << 4)
    for pos in rng.choice(n, live, replace=False):
        v.value[row[pos // 16], pos % 16] = rng.integers(0, 256, v.value.shape[-1:], dtype=np.uint8)


def test_planted_unrounded_zero_point_sum_fails_the_fp64_check(monkeypatch):
    """int4_kv.py:90-94: the zero-point correction must use the same bf16-rounded P * s_v as the PV product. With
    all but two keys' values at their zero points the true output is small, and the rounding gap of the unrounded
    variant (about 2^-9 of P s_v zp per key, over every key) dominates it."""
    for seed in (21, 22, 23):
        rng = np.random.default_rng(seed)
        n = 600
        v, row = _tiny_cache(rng, n, 2, 32, 16)
        _dead_values(rng, v, row, n, 2)
        q = O.round_bf16(rng.standard_normal((2, 4, 32)).astype(np.float32))
        K, V = O.dequant_f64(v, row, n)
        ref = O.attention_f64(q, K, V, n, 0.2)
        assert O.relerr(O.decode_emulated(q, v, row, n, 0.2, 2), ref) < 5e-3
        with monkeypatch.context() as mp:
            mp.setattr(O, "value_probabilities", lambda P, s, z: (O.round_bf16(P * s[None, :]),
                                                                  ((P * s[None, :]) * z[None, :]).sum(
                                                                      axis=1, dtype=np.float32)))
            assert O.relerr(O.decode_emulated(q, v, row, n, 0.2, 2), ref) > 3e-2


def test_max_row_relerr_hand_rows():
    ref = np.array([[[3.0, 4.0], [1.0, 0.0]]])            # two rows of head size 2, norms 5 and 1
    o = ref.copy()
    o[0, 0, 0] += 0.05                                     # row 0: 0.05 / 5 = 1 %
    o[0, 1, 1] += 0.03                                     # row 1: 0.03 / 1 = 3 %
    assert abs(O.max_row_relerr(o, ref) - 0.03) < 1e-12
    assert O.relerr(o, ref) < 0.03                         # the Frobenius figure hides row 1


# The oracle's int4 store assumes v * inv + zp is one fused multiply-add (k8v4_ops.py:55-56). These rows (min, max,
# probe), all bf16 values, put the probe within an ulp of a rounding boundary, where a mul-then-add store would pick the
# other code.
FMA_ROWS = [(-2.5625, 2.28125, -1.453125, 3, 4), (-2.671875, 2.171875, -1.453125, 3, 4),
            (-0.61328125, 0.30859375, -0.4609375, 2, 3), (-2.515625, 2.171875, -2.34375, 0, 1)]   # bf16-exact


def fma_rows(hs):
    """[len(FMA_ROWS), hs] fp32 rows: min, max, the probe, then zeros; and the probe's FMA code per row."""
    x = np.zeros((len(FMA_ROWS), hs), np.float32)
    for i, (lo, hi, probe, _, _) in enumerate(FMA_ROWS):
        x[i, :3] = (lo, hi, probe)
    return x, np.array([r[3] for r in FMA_ROWS])


def test_store_takes_the_fused_multiply_add_code():
    x, want = fma_rows(16)
    codes, _ = O.quantize_int4(x)
    got = codes[:, 1] & 0xF                                 # channel 2 = low nibble of byte 1
    assert (got == want).all()
    for lo, hi, probe, fma_code, muladd_code in FMA_ROWS:   # the two roundings do differ on these probes
        scale = np.maximum((np.float32(hi) - np.float32(lo)) / np.float32(15.0), np.float32(1e-6))
        zp = np.clip(O.round_half_away(-np.float32(lo) / scale), 0, 15).astype(np.float32)
        inv = np.float32(1.0) / scale
        assert O.round_half_away(np.float32(probe) * inv + zp) == muladd_code != fma_code


# ----------------------------------------------------------------- single-kernel int8 prefill (a14, _attn_i8)

def test_quantize_query_i8_known_answers():
    """int4_prefill.py:181-189 by hand on a row whose scale is 1 (max |q| = 127 in log2 units): hi = round half to
    even, lo = the rounded remainder in 1/254 units, q_sum = sum(hi) * 254 + sum(lo); a zero row takes the 1e-20 floor
    and splits to zeros."""
    scale = 1.0 / O.LOG2E                       # f32(scale * LOG2E) == 1.0
    row = [127.0, 1.5, -2.25, 0.5, 3.75, -0.5, 0.0, -127.0]
    q = np.array([row, [0.0] * 8], np.float32)[None]                      # [1 token, 2 heads, 8]
    hi, lo, qs, q_sum = O.quantize_query_i8(O.f32_to_bf16_bits(q), scale)
    assert qs[0, 0] == np.float32(1.0)
    assert hi[0, 0].tolist() == [127, 2, -2, 0, 4, 0, 0, -127]
    assert lo[0, 0].tolist() == [0, -127, -64, 127, -64, -127, 0, 0]    # -63.5 -> -64 (half to even)
    assert q_sum[0, 0] == (127 + 2 - 2 + 4 - 127) * 254 + (-127 - 64 + 127 - 64 - 127)
    assert qs[0, 1] == np.float32(1e-20) and not hi[0, 1].any() and not lo[0, 1].any() and q_sum[0, 1] == 0


def test_quantize_query_i8_reconstructs_and_matches_torch():
    """q ~ q_scale (hi + lo / 254) within half a 1/254 step (plus fp32 rounding); and torch running the reference's
    own lines (int4_prefill.py:181-189) gives the same integers and scales bit for bit."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    bits = O.f32_to_bf16_bits((rng.standard_normal((16, 6, 64)) * rng.lognormal(0, 1, (16, 6, 1))).astype(np.float32))
    scale = 64 ** -0.5
    hi, lo, qs, q_sum = O.quantize_query_i8(bits, scale)
    q = O.bf16_bits_to_f32(bits).astype(np.float64) * np.float32(scale * O.LOG2E)
    rec = qs[..., None].astype(np.float64) * (hi + lo / 254.0)
    assert (np.abs(q - rec) <= qs[..., None] * (0.5 / 254 + 1e-5)).all()
    tq = torch.from_numpy(O.bf16_bits_to_f32(bits)).float() * (scale * O.LOG2E)
    t_scale = (tq.abs().amax(-1) / 127.0).clamp_min(1e-20)
    tn = tq / t_scale[..., None]
    t_hi = torch.round(tn)
    t_lo = torch.round((tn - t_hi) * 254).clamp(-127, 127)
    t_sum = (t_hi.sum(-1) * 254 + t_lo.sum(-1)).to(torch.int32)
    assert (t_scale.numpy() == qs).all()
    assert (t_hi.to(torch.int8).numpy() == hi).all() and (t_lo.to(torch.int8).numpy() == lo).all()
    assert (t_sum.numpy() == q_sum).all()


def test_i8_scores_brute_force():
    """Integer dots and the two fp32 products of int4_prefill.py:136-138, term by term on a tiny case."""
    rng = np.random.default_rng(22)
    v, row = _tiny_cache(rng, 5, 1, 8, 16)
    bits = O.f32_to_bf16_bits(rng.standard_normal((2, 1, 8)).astype(np.float32))
    hi, lo, qs, q_sum = O.quantize_query_i8(bits, 0.3)
    kc, kw, _, _ = O.gather(v, row, np.arange(5))
    got = O.i8_scores(hi[:, 0], lo[:, 0], q_sum[:, 0], qs[:, 0], kc[:, 0], kw[:, 0])
    for t in range(2):
        for j in range(5):
            codes = [(int(kc[j, 0, c // 2]) >> (4 * (c % 2))) & 0xF for c in range(8)]
            w = int(kw[j, 0])
            dot = sum((int(hi[t, 0, c]) * 254 + int(lo[t, 0, c])) * codes[c] for c in range(8)) - int(q_sum[t, 0]) * (w & 0xF)
            ks = np.uint32(w & 0xFFFFFFF0).view(np.float32)
            want = np.float32(np.float32(dot) * np.float32(qs[t, 0] / np.float32(254))) * ks
            assert got[t, j] == want, (t, j)


def _i8_case(seed=23, T=48, n=600, nq=6, nkv=2, hs=32):
    rng = np.random.default_rng(seed)
    v, row = _tiny_cache(rng, n, nkv, hs, 16)
    q = O.round_bf16(rng.standard_normal((T, nq, hs)).astype(np.float32))
    K, V = O.dequant_f64(v, row, n)
    return v, row, q, O.attention_f64(q, K, V, n, hs ** -0.5)


def test_prefill_i8_emulated_matches_fp64():
    v, row, q, ref = _i8_case()
    got = O.prefill_i8_emulated(O.f32_to_bf16_bits(q), v, row, 600, 32 ** -0.5)
    assert O.relerr(got, ref) < 2e-3 and O.max_row_relerr(got, ref) < 5e-3


@pytest.mark.parametrize("kind", ["hi-only", "no-key-zero-point", "no-value-zero-point", "q-sum-weight-256"])
def test_prefill_i8_planted_mistakes_fail_the_fp64_check(monkeypatch, kind):
    """Each variant departs from int4_prefill.py:136-165 in one term and must fail the check the real one passes.
    hi-only is the one-int8 split whose error the reference's docstring puts at about 1.3e-2 (:104-105)."""
    v, row, q, ref = _i8_case(seed=24)
    bits = O.f32_to_bf16_bits(q)
    good = O.relerr(O.prefill_i8_emulated(bits, v, row, 600, 32 ** -0.5), ref)
    real_q, real_parts, real_scores = O.quantize_query_i8, O.int4_word_parts, O.i8_scores
    if kind == "hi-only":
        monkeypatch.setattr(O, "quantize_query_i8", lambda b, s: (lambda h, l, qs, sm: (
            h, np.zeros_like(l), qs, h.astype(np.int64).sum(-1) * O.Q_LO))(*real_q(b, s)))
    elif kind == "no-key-zero-point":
        monkeypatch.setattr(O, "i8_scores", lambda hi, lo, sm, qs, kc, kw: real_scores(
            hi, lo, np.zeros_like(sm), qs, kc, kw))
    elif kind == "no-value-zero-point":
        calls = {"n": 0}

        def parts(w):
            calls["n"] += 1
            zp, sc = real_parts(w)
            return (np.zeros_like(zp) if calls["n"] % 2 == 1 else zp), sc   # the value half's call comes first
        monkeypatch.setattr(O, "int4_word_parts", parts)
    elif kind == "q-sum-weight-256":  # the zero-point term's query sum with the hi part weighted 256, not 254
        monkeypatch.setattr(O, "quantize_query_i8", lambda b, s: (lambda h, l, qs, sm: (
            h, l, qs, h.astype(np.int64).sum(-1) * 256 + l.astype(np.int64).sum(-1)))(*real_q(b, s)))
    bad = O.relerr(O.prefill_i8_emulated(bits, v, row, 600, 32 ** -0.5), ref)
    assert good < 2e-3 and bad > 4 * good, (good, bad)
