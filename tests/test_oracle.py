"""Pins the CPU oracle (oracle/oracle.c) against the reference's golden vectors, against
an independent library (numpy's IEEE float16), and against what the mathematics fixes."""
import json
import math
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))


def test_f16_to_f32_every_pattern_matches_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_values(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN payloads are kept (quiet bit and top payload bits), as formats.rs does
    assert np.array_equal(got[nan].view(np.uint32) >> 13 & 0x3FF, h[nan] & 0x3FF)


def test_f32_to_f16_round_trips_every_f16():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = h.view(np.float16).astype(np.float32)
    back = oracle.f16_bits(x)
    finite = ~np.isnan(x)
    assert np.array_equal(back[finite], h[finite])
    assert np.all((back[~finite] & 0x7C00) == 0x7C00) and np.all(back[~finite] & 0x3FF)


def test_f32_to_f16_is_ieee_rne_like_numpy():
    r = np.random.default_rng(1)
    # every exponent, random mantissas, both signs
    bits = r.integers(0, 2**32, 2**21, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f16_bits(x), want)
    # dense around the subnormal/normal boundary and the overflow threshold
    for lo, hi in [(0.0, 1.3e-4), (65000.0, 66000.0), (5.0e-8, 7.0e-8)]:
        y = np.linspace(lo, hi, 200001, dtype=np.float32)
        y = np.concatenate([y, -y])
        with np.errstate(over="ignore"):
            assert np.array_equal(oracle.f16_bits(y), y.astype(np.float16).view(np.uint16))


def test_f32_to_f16_halfway_cases_round_to_even():
    # Midpoints between consecutive positive finite f16 values are exact in f32.
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    a = h.view(np.float16).astype(np.float64)
    b = (h + 1).view(np.float16).astype(np.float64)
    mid = ((a + b) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (a + b) / 2)
    got = oracle.f16_bits(mid)
    want = np.where(h % 2 == 0, h, h + 1).astype(np.uint16)
    assert np.array_equal(got, want)


def test_fixture_narrowing_equals_rne_on_normals_and_flushes_below():
    """xtask/src/fixtures.rs:45-67 flushes f16 subnormals; the KV store keeps them."""
    r = np.random.default_rng(2)
    x = (r.standard_normal(20000) * 100).astype(np.float32)
    x = x[np.abs(x) >= 6.103515625e-05]
    assert all(oracle.f32_to_f16_fixture(float(v)) == oracle.f32_to_f16(float(v)) for v in x[:5000])
    assert oracle.f32_to_f16_fixture(1e-6) == 0 and oracle.f32_to_f16(1e-6) != 0
    assert oracle.f32_to_f16_fixture(-1e-6) == 0x8000


def _golden_q8():
    with open(os.path.join(HERE, "golden", "ggml_dequant_q8_0.json")) as f:
        c = json.load(f)["case"]
    raw = np.frombuffer(bytes.fromhex(c["bytes_hex"]), np.uint8)
    want = np.array(c["f32_bits"], np.uint64).astype(np.uint32)
    return raw, want, c["cols"]


def test_q8_0_dequant_matches_gguf_py_golden_vector():
    """fixtures/oracle/ggml_dequant.json (gguf-py 0.19.0), bit for bit, as
    crates/qubivex-backend-cpu/tests/oracle.rs:10-50 checks it."""
    raw, want, cols = _golden_q8()
    got = oracle.q8_0_dequant(raw, cols)
    assert np.array_equal(got.view(np.uint32), want)


def test_q8_0_dequant_rejects_a_dropped_factor():
    """Positive control: dequant without the scale must not match the golden vector."""
    raw, want, cols = _golden_q8()
    plain = raw.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.float32).reshape(-1)
    assert not np.array_equal(plain.view(np.uint32), want)


def q8_blocks(q):
    q = np.asarray(q, np.uint8).reshape(-1, 34)
    scale = q[:, 0].astype(np.uint16) | (q[:, 1].astype(np.uint16) << 8)
    return scale, q[:, 2:].view(np.int8)


def test_q8_0_quantize_closed_forms():
    # all zeros: scale 0, values 0
    s, v = q8_blocks(oracle.q8_0_quantize(np.zeros(32, np.float32)))
    assert s[0] == 0 and not v.any()
    # amax 127 gives d = 1 exactly: x*inv = x; ties go away from zero
    x = np.zeros(32, np.float32)
    x[:8] = [127, -127, 2.5, -2.5, 0.5, -0.5, 3.49, -3.51]
    s, v = q8_blocks(oracle.q8_0_quantize(x))
    assert s[0] == 0x3C00  # f16(1.0)
    assert v[0, :8].tolist() == [127, -127, 3, -3, 1, -1, 3, -4]
    # +-amax always quantizes to +-127 and the scale is f16(amax/127)
    r = np.random.default_rng(3)
    for _ in range(200):
        y = r.standard_normal(32).astype(np.float32)
        i = int(np.argmax(np.abs(y)))
        s, v = q8_blocks(oracle.q8_0_quantize(y))
        assert abs(int(v[0, i])) == 127 and np.sign(v[0, i]) == np.sign(y[i])
        d = np.float32(np.max(np.abs(y))) / np.float32(127)
        assert s[0] == np.float16(d).view(np.uint16)
    # NaN is ignored by the maximum and quantizes to 0
    y = np.ones(32, np.float32)
    y[3] = np.nan
    s, v = q8_blocks(oracle.q8_0_quantize(y))
    assert v[0, 3] == 0 and v[0, 0] == 127
    # inf: the scale overflows to inf, inv = 0, every value 0 (inf*0 = NaN -> 0)
    y = np.ones(32, np.float32)
    y[5] = np.inf
    s, v = q8_blocks(oracle.q8_0_quantize(y))
    assert s[0] == 0x7C00 and not v.any()


def test_q8_0_quantize_uses_the_f32_scale_not_the_rounded_one():
    """inv comes from the f32 d (fixtures.rs:80).  Pick amax where f16 rounding of d
    changes round(x*inv) for some x: the oracle must follow the f32 d."""
    r = np.random.default_rng(4)
    found = 0
    for _ in range(2000):
        y = (r.standard_normal(32) * 3).astype(np.float32)
        s, v = q8_blocks(oracle.q8_0_quantize(y))
        d32 = np.float32(np.max(np.abs(y))) / np.float32(127)
        from_f32 = np.clip(np.round(y * (np.float32(1) / d32) + 0), -127, 127)
        d16 = np.float32(np.float16(d32))
        from_f16 = np.clip(np.round(y * (np.float32(1) / d16)), -127, 127)
        if not np.array_equal(from_f32, from_f16):
            found += 1
            # numpy rounds half to even; exclude exact ties (measure zero here)
            assert np.array_equal(v[0].astype(np.float32), from_f32)
    assert found > 0


def test_q8_0_round_trip_error_is_bounded_by_half_a_step():
    r = np.random.default_rng(5)
    x = r.standard_normal(32 * 512).astype(np.float32)
    x[r.random(x.size) < 0.01] *= 8
    y = oracle.q8_0_dequant(oracle.q8_0_quantize(x), x.size)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
    d16 = np.float16(amax / 127).astype(np.float32)
    err = np.abs(y.reshape(-1, 32) - x.reshape(-1, 32))
    # |q*d16 - x| <= d32/2 + 127*|d16 - d32| (the scale's own rounding)
    bound = amax / 127 / 2 + 127 * np.abs(d16 - amax / 127) + 1e-7
    assert np.all(err <= bound)


def test_q8_0_requantizing_golden_blocks_is_idempotent():
    raw, _, cols = _golden_q8()
    blocks = raw.reshape(-1, 34)
    checked = 0
    for b in blocks:
        q = b[2:].view(np.int8)
        if q.min() < -127 or np.abs(q.astype(int)).max() != 127:
            continue
        y = oracle.q8_0_dequant(b.copy(), 32)
        again = oracle.q8_0_quantize(y)
        assert np.array_equal(again[2:].view(np.int8), q)
        checked += 1
    # random golden bytes rarely have |q| max == 127 without -128; construct one
    s = np.float16(0.0123).view(np.uint16)
    q = np.random.default_rng(6).integers(-126, 127, 32).astype(np.int8)
    q[7] = -127
    b = np.concatenate([[s & 0xFF, s >> 8], q.view(np.uint8)]).astype(np.uint8)
    again = oracle.q8_0_quantize(oracle.q8_0_dequant(b, 32))
    assert np.array_equal(again[2:].view(np.int8), q)
    assert int(again[0]) | (int(again[1]) << 8) == int(s)


def _ulps(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


def test_exp_within_two_ulp_over_the_normal_range():
    """crates/qubivex-compute/src/math.rs:187-208, the reference's own sweep."""
    xs = []
    x = -87.33655
    while x < 88.72284:
        xs.append(x)
        x += max(abs(x) * 1e-5, 1e-6)
    xs = np.array(xs, np.float32)
    want = np.exp(xs.astype(np.float64))
    ok = (want >= np.finfo(np.float32).tiny) & (want <= np.finfo(np.float32).max)
    got = oracle.exp_vec(xs[ok])
    assert xs.size > 1_500_000
    assert _ulps(got, want[ok].astype(np.float32)).max() <= 2


def test_exp_edges():
    """math.rs:210-228."""
    assert oracle.exp(0.0) == 1.0 and oracle.exp(-0.0) == 1.0
    assert math.isnan(oracle.exp(float("nan")))
    assert oracle.exp(float("inf")) == float("inf")
    assert oracle.exp(float("-inf")) == 0.0
    assert oracle.exp(100.0) == float("inf") and oracle.exp(-100.0) == 0.0
    assert oracle.exp(-87.5) == 0.0
    assert oracle.exp(88.7) < float("inf")
    assert oracle.exp(-87.3365) >= np.finfo(np.float32).tiny
    assert abs(oracle.exp(1.0) - math.e) <= 4 * np.finfo(np.float32).eps


def test_softmax_sums_to_one_and_keeps_order():
    r = np.random.default_rng(7)
    x = (r.standard_normal(1000) * 5).astype(np.float32)
    p = oracle.softmax(x)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.array_equal(np.argsort(p, kind="stable"), np.argsort(x, kind="stable"))


def test_attend_special_cases_and_f64_agreement():
    r = np.random.default_rng(8)
    d = 64
    for n in [1, 2, 17, 500]:
        q = r.standard_normal(d).astype(np.float32)
        k = r.standard_normal((n, d)).astype(np.float32)
        v = r.standard_normal((n, d)).astype(np.float32)
        got = oracle.attend(q, k, v, n - 1)
        want = oracle.attend_f64(q, k, v, n - 1)
        assert np.max(np.abs(got - want)) < 1e-5
        if n == 1:
            assert np.array_equal(got, v[0])  # one position: exactly v_0
    # equal scores (zero query): the mean of the values
    q = np.zeros(d, np.float32)
    k = r.standard_normal((40, d)).astype(np.float32)
    v = r.standard_normal((40, d)).astype(np.float32)
    np.testing.assert_allclose(oracle.attend(q, k, v, 39), v.mean(axis=0), atol=1e-6)
    # a one-hot query with a huge weight picks the key with the largest coordinate
    q = np.zeros(d, np.float32)
    q[5] = 1000.0
    got = oracle.attend(q, k, v, 39)
    np.testing.assert_allclose(got, v[np.argmax(k[:, 5])], atol=1e-5)


def test_attend_positive_control_wrong_scale_is_caught():
    r = np.random.default_rng(9)
    d, n = 128, 300
    q = r.standard_normal(d).astype(np.float32)
    k = r.standard_normal((n, d)).astype(np.float32)
    v = r.standard_normal((n, d)).astype(np.float32)
    got = oracle.attend(q, k, v, n - 1)
    wrong = oracle.attend(q * np.float32(np.sqrt(d)), k, v, n - 1)  # scale dropped
    assert np.max(np.abs(got - wrong)) > 1e-2


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.Q8_0])
def test_sim_pool_store_gather_round_trip(dtype):
    r = np.random.default_rng(10)
    G, d, B = 2, 64, 16
    sim = oracle.SimPool(12, G, d, B, dtype)
    n = 40
    blocks = r.permutation(12)[:3].astype(np.uint32)
    table_at = np.array([0], np.uint32)
    slots = (blocks[np.arange(n) // B].astype(np.int64) * B + np.arange(n) % B).astype(np.uint32)
    k = r.standard_normal((n, G * d)).astype(np.float32)
    v = r.standard_normal((n, G * d)).astype(np.float32)
    sim.store(k, v, slots)
    gk, gv = sim.gather(blocks, table_at, 0, n)
    if dtype == oracle.F16:
        wk = k.astype(np.float16).astype(np.float32)
        wv = v.astype(np.float16).astype(np.float32)
    else:
        wk = np.stack([oracle.q8_0_dequant(oracle.q8_0_quantize(row), G * d) for row in k])
        wv = np.stack([oracle.q8_0_dequant(oracle.q8_0_quantize(row), G * d) for row in v])
    assert np.array_equal(gk, wk.reshape(n, G, d).transpose(1, 0, 2))
    assert np.array_equal(gv, wv.reshape(n, G, d).transpose(1, 0, 2))


def test_reference_layout_addressing_at_block_256():
    """discrete.rs:247-255,319-329 at KV_BLOCK = 256: keys dimension-major then values
    position-major, every word of a block hit exactly once."""
    G, d, B = 2, 8, 256
    kv_out = G * d
    words = set()
    L = oracle.lib()
    for at in range(B, 2 * B):  # block 1
        for g in range(G):
            for i in range(d):
                words.add(L.orc_key_word(kv_out, d, B, at, g, i))
                words.add(L.orc_value_word(kv_out, d, B, at, g, i))
    assert words == set(range(2 * B * kv_out, 4 * B * kv_out))
    assert L.orc_key_word(kv_out, d, B, B + 3, 1, 2) == 2 * B * kv_out + (1 * d + 2) * B + 3
    assert L.orc_value_word(kv_out, d, B, B + 3, 1, 2) == 2 * B * kv_out + B * kv_out + 3 * kv_out + d + 2


def test_reduce_dot_matches_f64_and_handles_tails():
    """crates/qubivex-compute/src/reduce.rs:56-80, the reference's own test."""
    for n in [0, 1, 31, 32, 63, 64, 65, 100, 128, 1000, 2048]:
        i = np.arange(n)
        w = (((i * 37) % 101).astype(np.float32) - 50) / np.float32(64)
        x = (((i * 53) % 97).astype(np.float32) - 48) / np.float32(32)
        want = float(np.sum(w.astype(np.float64) * x.astype(np.float64)))
        got = oracle.reduce_dot(w, x)
        assert abs(got - want) <= 1e-5 * max(abs(want), 1.0), (n, got, want)


def _lanes(vals, n=64):
    """A 64-element vector with the given {lane: value}; dot with ones puts each value in
    its accumulator lane exactly (fma(v, 1, 0) = v)."""
    w = np.zeros(n, np.float32)
    for lane, v in vals.items():
        w[lane] = v
    return w


# Hand-computed pins of reduce.rs:14-50's tree (a[i] += a[i + w] for w = 32, 16, 8, 4, then
# (a0 + a1) + (a2 + a3)), all in f32 where 1e8 + 1 rounds back to 1e8 (ulp 8) and
# 2^24 + 1 ties to 2^24.  Each expected value was worked out by hand from that tree; the
# comment gives what another pairing or order gives instead.
REDUCE_PINS = [
    # final stage: (1e8 + 1) + (-1e8 + 1) = 1e8 - 1e8 = 0; sequential 1, (a0+a2)+(a1+a3) 2
    (_lanes({0: 1e8, 1: 1, 2: -1e8, 3: 1}), 0.0),
    # stage w pairs lane 0 with w and 1 with w + 1: a0 = 0, a1 = 2, so 2; adjacent pairs
    # (0 with 1) absorb the ones into +-1e8 and give 0, a sequential sum 1
    (_lanes({0: 1e8, 1: 1, 32: -1e8, 33: 1}), 2.0),
    (_lanes({0: 1e8, 1: 1, 16: -1e8, 17: 1}), 2.0),
    (_lanes({0: 1e8, 1: 1, 8: -1e8, 9: 1}), 2.0),
    (_lanes({0: 1e8, 1: 1, 4: -1e8, 5: 1}), 2.0),
    # stage order: w = 32 first adds lane 32 into 0 and 48 into 16, absorbing both ones:
    # (1e8 + 1) + (-1e8 + 1) = 0; w = 16 first (or a sequential sum) gives 2
    (_lanes({0: 1e8, 16: -1e8, 32: 1, 48: 1}), 0.0),
    # all positive (a sum of squares, as in rms_norm): (2^24 + 1) + (1 + 1) = 2^24 + 2;
    # sequential 2^24 (each 1 ties back to 2^24)
    (_lanes({0: 2.0 ** 24, 1: 1, 2: 1, 3: 1}), 2.0 ** 24 + 2),
    # tail of a 65-element vector: element 64 goes to lane 0 (lanes 0..rem): lane 0 =
    # 1e8 + 1 = 1e8, so (1e8 - 1e8) + (1 + 0) = 1; tail in lane 2 gives 2, sequential 2
    (np.concatenate([_lanes({0: 1e8, 1: -1e8, 2: 1}), np.float32([1])]), 1.0),
]


@pytest.mark.parametrize("w,want", REDUCE_PINS, ids=range(len(REDUCE_PINS)))
def test_reduce_dot_tree_order_pinned_by_hand(w, want):
    got = oracle.reduce_dot(w, np.ones_like(w))
    assert got == want, (got, want)
    # the same values split between w and x (w * x, exact products) give the same bits
    assert oracle.reduce_dot(w * 2, np.full_like(w, 0.5)) == want


def test_reduce_dot_pins_reject_other_trees():
    """Positive control: each plausible wrong reduction (sequential, adjacent pairs,
    stages in increasing width) misses at least one pin above."""
    def tree(a, widths, final):
        a = a.astype(np.float32).copy()
        for wd in widths:
            for i in range(wd):
                a[i] = np.float32(a[i] + a[i + wd])
        return float(final(a))

    def lanes_of(w):
        acc = np.zeros(64, np.float32)
        for i, v in enumerate(w):
            acc[i % 64] = np.float32(acc[i % 64] + v)
        return acc

    def seq(w):
        s = np.float32(0)
        for v in w:
            s = np.float32(s + v)
        return float(s)

    ref_final = lambda a: np.float32(np.float32(a[0] + a[1]) + np.float32(a[2] + a[3]))  # noqa: E731
    wrong = {
        "sequential": seq,
        "increasing widths": lambda w: tree(lanes_of(w), [4, 8, 16, 32], ref_final),
        "final (a0+a2)+(a1+a3)": lambda w: tree(
            lanes_of(w), [32, 16, 8, 4],
            lambda a: np.float32(np.float32(a[0] + a[2]) + np.float32(a[1] + a[3]))),
        "final sequential": lambda w: tree(
            lanes_of(w), [32, 16, 8, 4],
            lambda a: np.float32(np.float32(np.float32(a[0] + a[1]) + a[2]) + a[3])),
        "down to 1 lane": lambda w: tree(lanes_of(w), [32, 16, 8, 4, 2, 1], lambda a: a[0]),
    }
    right = lambda w: tree(lanes_of(w), [32, 16, 8, 4], ref_final)  # noqa: E731
    for w, want in REDUCE_PINS:
        assert right(w) == want  # the hand values are the tree's
    for name, f in wrong.items():
        assert any(f(w) != want for w, want in REDUCE_PINS), name


def test_reduce_dot_shape_is_observable():
    """Positive control: a plain sequential sum gives other bits on some inputs, so a
    kernel that matches the shape bit for bit does follow it."""
    r = np.random.default_rng(12)
    differ = 0
    for _ in range(200):
        x = (r.standard_normal(4096) * 10).astype(np.float32)
        seq = np.float32(0)
        for v in x:
            seq = np.float32(np.fma(v, v, seq)) if hasattr(np, "fma") else np.float32(seq + v * v)
        differ += oracle.reduce_dot(x, x) != float(seq)
        if differ:
            break
    assert differ


def test_rms_norm_and_rope_closed_forms():
    # 64 threes: ss = 576 exactly, ss/n = 9, sqrt = 3, r = f32(1/3)
    y = oracle.rms_norm(np.full(64, 3.0, np.float32), np.ones(64, np.float32), 0.0)
    assert np.all(y == np.float32(3.0) * (np.float32(1.0) / np.float32(3.0)))
    # the weights multiply after the scale
    w = np.arange(64, dtype=np.float32)
    y2 = oracle.rms_norm(np.full(64, 3.0, np.float32), w, 0.0)
    assert np.array_equal(y2, y * w)
    r = np.random.default_rng(13)
    h = r.standard_normal(128).astype(np.float32)
    ident = np.concatenate([np.ones(64), np.zeros(64)]).astype(np.float32)
    assert np.array_equal(oracle.rope_rotate(h, ident), h)
    quarter = np.concatenate([np.zeros(64), np.ones(64)]).astype(np.float32)
    assert np.array_equal(oracle.rope_rotate(h, quarter), np.concatenate([-h[64:], h[:64]]))
    # a rotation keeps each pair's length (to rounding)
    a = r.uniform(0, 6.3, 64)
    cs = np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32)
    y = oracle.rope_rotate(h, cs)
    np.testing.assert_allclose(y[:64] ** 2 + y[64:] ** 2, h[:64] ** 2 + h[64:] ** 2, rtol=1e-5)


def test_prelude_composes_bias_clip_norm_rope_in_order():
    r = np.random.default_rng(14)
    heads, kvh, d, s = 4, 2, 64, 3
    q = (r.standard_normal((s, heads * d)) * 3).astype(np.float32)
    k = (r.standard_normal((s, kvh * d)) * 3).astype(np.float32)
    v = (r.standard_normal((s, kvh * d)) * 3).astype(np.float32)
    rope = r.uniform(-1, 1, (s, d)).astype(np.float32)
    qb = r.standard_normal(heads * d).astype(np.float32)
    qn = r.uniform(0.5, 1.5, d).astype(np.float32)
    kn = r.uniform(0.5, 1.5, d).astype(np.float32)
    gq, gk, gv = oracle.prelude(q, k, v, heads, kvh, d, rope, q_bias=qb, clip=2.5, norm=2,
                                q_norm=qn, k_norm=kn, eps=1e-6)
    # by hand with the single-step functions
    wq = np.clip(q + qb, -2.5, 2.5).astype(np.float32)
    wk = np.clip(k, -2.5, 2.5).astype(np.float32)
    for t in range(s):
        for h in range(heads):
            x = oracle.rms_norm(wq[t, h * d:(h + 1) * d], qn, 1e-6)
            wq[t, h * d:(h + 1) * d] = oracle.rope_rotate(x, rope[t])
        for h in range(kvh):
            x = oracle.rms_norm(wk[t, h * d:(h + 1) * d], kn, 1e-6)
            wk[t, h * d:(h + 1) * d] = oracle.rope_rotate(x, rope[t])
    assert np.array_equal(gq.reshape(s, -1), wq) and np.array_equal(gk.reshape(s, -1), wk)
    assert np.array_equal(gv.reshape(s, -1), np.clip(v, -2.5, 2.5))
