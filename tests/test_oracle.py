"""CPU pins of the oracle: the reference's known answers, two independent restatements that must agree, and
closed forms. A check that fails when a plausible mistake is planted in the oracle is included for each
family (test_planted_*)."""

import json
import math
import os

import numpy as np
import pytest

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def _f(v):
    return float(v) if not isinstance(v, str) else float(v.replace("inf", "inf"))


# ---- 16-bit floats ------------------------------------------------------------------------------------

def test_bf16_ties_and_nonfinite(oracle):
    ka = GOLDEN["bf16_ties_and_nonfinite"]
    vals = np.array([_f(v) for v in ka["values"]], np.float32)
    got = oracle.bf16_round(vals)
    exp = np.array([_f(v) for v in ka["expected"]], np.float32)
    np.testing.assert_array_equal(got[:5], exp[:5])
    assert np.isnan(got[5])


def test_bf16_scale_tie_bits(oracle):
    ka = GOLDEN["scale_tie_bits"]
    vals = np.array(ka["input_bits"], np.uint32).view(np.float32)
    np.testing.assert_array_equal(oracle.bf16_bits(vals), np.array(ka["expected_bf16_bits"], np.uint16))


def test_f16_rounding_matches_ieee_cast(oracle):
    # numpy's float32 -> float16 cast is IEEE round-to-nearest-even; the C restatement must match it everywhere,
    # including subnormals, overflow and ties.
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300000) * np.exp(rng.uniform(-30, 13, 300000))).astype(np.float32)
    ties = (np.arange(1, 2049, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)  # halfway cases near 1..3
    special = np.array([65504, 65519.99, 65520, 6.103515625e-05, 5.960464477539063e-08, 2.98e-8, 2.99e-8, 0.0, -0.0,
                        np.inf, -np.inf], np.float32)
    allv = np.concatenate([x, -x, ties, special])
    with np.errstate(over="ignore"):
        ref = allv.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f16_bits(allv), ref)


def test_bf16_rounding_matches_closed_form(oracle):
    # Round-to-nearest-even on the upper 16 bits, checked against float64 arithmetic on the candidates.
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-20, 20, 100000))).astype(np.float32)
    got = oracle.bf16_round(x).astype(np.float64)
    bits = x.view(np.uint32)
    lo = (bits & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi_bits = (bits & 0xFFFF0000) + 0x10000
    hi = hi_bits.astype(np.uint32).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    d_lo, d_hi = np.abs(xd - lo), np.abs(hi - xd)
    even_lo = ((bits >> 16) & 1) == 0
    exp = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(even_lo, lo, hi)))
    np.testing.assert_array_equal(got, exp)


# ---- portable nibble order and dequantization --------------------------------------------------------

def test_nibble_order_and_group_dequant(oracle):
    ka = GOLDEN["nibble_order_and_group_dequant"]
    q = np.array(ka["q"], np.uint8)
    packed = oracle.pack_int4(q)
    np.testing.assert_array_equal(packed, np.array(ka["packed"], np.uint8))
    np.testing.assert_array_equal(oracle.unpack_int4(packed), q)
    deq = oracle.dequantize_portable(packed, np.array(ka["scales"]), np.array(ka["zeros"]), ka["group"])
    np.testing.assert_array_equal(deq, np.array(ka["dequant"]))
    # The logical [K, N] dequantizer is the transpose of the portable one.
    np.testing.assert_array_equal(oracle.dequantize(q.T, np.array(ka["scales"]).T, np.array(ka["zeros"]).T, ka["group"]),
                                  np.array(ka["dequant"]).T)


def test_unsigned_zero_points(oracle):
    ka = GOLDEN["zero_points_unsigned"]
    w = oracle.dequantize(np.full((128, 64), ka["q"], np.uint8), np.full((1, 64), ka["scale"]), np.full((1, 64), ka["zero"], np.uint8), 128)
    assert np.all(w == ka["expected"])


def test_planted_dequant_mistake_is_caught(oracle):
    # Swapping q and z, or dropping the zero, must break the known answer.
    ka = GOLDEN["nibble_order_and_group_dequant"]
    q = np.array(ka["q"], np.float64)
    s = np.repeat(np.array(ka["scales"], np.float64), 2, axis=1)
    z = np.repeat(np.array(ka["zeros"], np.float64), 2, axis=1)
    exp = np.array(ka["dequant"])
    assert not np.array_equal((z - q) * s, exp)
    assert not np.array_equal(q * s, exp)


# ---- SwiGLU rounding ----------------------------------------------------------------------------------

def test_silu_bf16_double_rounding(oracle):
    ka = GOLDEN["bf16_silu_double_rounding"]
    gate = np.array(ka["gate"], np.float32)
    up = np.full_like(gate, ka["up"])
    got = oracle.silu_multiply_bf16_io(gate, up)
    np.testing.assert_array_equal(got, np.array(ka["expected"], np.float32))
    single = oracle.bf16_round((oracle.silu(gate) * up).astype(np.float32))
    for i in ka["single_rounding_differs_at"]:
        assert single[i] != got[i]


def test_silu_stable_extremes(oracle):
    v = oracle.silu(np.array([-1000.0, -1.0, 0.0, 1.0, 1000.0]))
    np.testing.assert_allclose(v, [0.0, -1 / (1 + math.e), 0.0, 1 / (1 + math.exp(-1)), 1000.0], atol=1e-12)


# ---- 4352-byte tiles ------------------------------------------------------------------------------

@pytest.mark.parametrize("k,n", [(128, 64), (128, 128), (384, 640), (256, 1152), (512, 1024)])
def test_pack_two_restatements_agree(oracle, k, n):
    rng = np.random.default_rng(k + n)
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.002, 0.02, 6, 10)
    np.testing.assert_array_equal(oracle.pack_tiles(q, s, z), oracle.pack_tiles_literal(q, s, z))


@pytest.mark.parametrize("k,n", [(128, 128), (384, 640), (256, 1152)])
def test_decoder_round_trip(oracle, k, n):
    # 10 and 18 tile columns: uneven column groups with a second column in some groups.
    rng = np.random.default_rng(7 * k + n)
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.003, 0.25, 0, 16)
    q2, s2, z2, zd = oracle.unpack_tiles(oracle.pack_tiles(q, s, z), k, n, with_dup=True)
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(s2, s)
    np.testing.assert_array_equal(z2, z)
    np.testing.assert_array_equal(zd, z)


def test_tile_index_closed_form(oracle):
    for tiles_k, tiles_n in [(1, 1), (3, 10), (32, 224), (112, 64), (2, 19)]:
        seen = set()
        for c in range(tiles_n):
            for r in range(tiles_k):
                before = c // 8 + sum((tiles_n - g + 7) // 8 for g in range(c % 8))
                idx = oracle.tile_index(c, r, tiles_k, tiles_n)
                assert idx == before * tiles_k + r
                seen.add(idx)
        assert seen == set(range(tiles_k * tiles_n))


def test_slices_are_tile_subsets(oracle):
    # check_packing.py:136-167: with split points at multiples of 512, an N-slice / K-slice packed alone is the
    # full buffer's tiles under a mask, in order.
    rng = np.random.default_rng(3)
    k, n, s0 = 256, 2048, 512
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.002, 0.02, 6, 10)
    full = oracle.pack_tiles(q, s, z).reshape(-1, 4352)
    order = [(c, r) for g in range(8) for c in range(g, n // 64, 8) for r in range(k // 128)]
    pos = {t: i for i, t in enumerate(order)}
    sub_order = [(c, r) for g in range(8) for c in range((n - s0) // 64) if c % 8 == g for r in range(k // 128)]
    sel = [pos[(c + s0 // 64, r)] for c, r in sub_order]
    got = oracle.pack_tiles(q[:, s0:], s[:, s0:], z[:, s0:]).reshape(-1, 4352)
    np.testing.assert_array_equal(got, full[sel])
    assert sel == sorted(sel)


def test_contract_sizes(oracle):
    ka = GOLDEN["contract_sizes"]
    assert (ka["hidden"] // 128) * (ka["intermediate"] // 64) * 4352 == ka["weight_bytes"]
    assert ka["m"] * ka["hidden"] * 2 == ka["activation_bytes"]
    assert ka["m"] * ka["npu_channels"] * 2 == ka["intermediate_bytes"]
    assert oracle.pack_tiles(np.zeros((128, 64), np.uint8), np.zeros((1, 64), np.uint16), np.zeros((1, 64), np.uint8)).size == 4352


def test_planted_tile_order_mistake_is_caught(oracle):
    # A packer that skips the column-group order (plain column-major tiles) disagrees with the decoder.
    rng = np.random.default_rng(4)
    k, n = 128, 640
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16")
    good = oracle.pack_tiles(q, s, z).reshape(-1, 4352)
    order = [(c, r) for g in range(8) for c in range(g, n // 64, 8) for r in range(k // 128)]
    plain = np.empty_like(good)
    for i, (c, r) in enumerate(order):
        plain[c * (k // 128) + r] = good[i]
    q2, _, _ = oracle.unpack_tiles(plain.ravel(), k, n)
    assert not np.array_equal(q2, q)


# ---- AWQ ----------------------------------------------------------------------------------------------

def test_awq_unpack_known_answer(oracle):
    # Word 0x76543210 holds nibble v at bits 4 v; AWQ order reads shifts 4 * [0, 4, 1, 5, 2, 6, 3, 7].
    packed = np.array([[0x76543210, 0x0000000F]], np.uint32).view(np.int32)
    got = oracle.awq_unpack(packed)
    np.testing.assert_array_equal(got[0, :8], [0, 4, 1, 5, 2, 6, 3, 7])
    np.testing.assert_array_equal(got[0, 8:], [15, 0, 0, 0, 0, 0, 0, 0])


def test_awq_unpack_is_a_permutation(oracle):
    rng = np.random.default_rng(5)
    packed = rng.integers(-2 ** 31, 2 ** 31, (4, 16), dtype=np.int64).astype(np.int32)
    got = oracle.awq_unpack(packed)
    words = packed.view(np.uint32)
    for j in range(16):
        nibbles = [(int(words[0, j]) >> (4 * i)) & 15 for i in range(8)]
        assert sorted(got[0, 8 * j:8 * j + 8]) == sorted(nibbles)
        assert [got[0, 8 * j + k] for k in range(8)] == [nibbles[i] for i in (0, 4, 1, 5, 2, 6, 3, 7)]


# ---- GEMV / FFN closed forms ----------------------------------------------------------------------

def test_constant_input_gives_exactly_eight(oracle):
    ka = GOLDEN["constant_input"]
    k = ka["k"]
    x = np.full((1, k), ka["x"])
    w = oracle.dequantize(np.full((k, 64), ka["q"], np.uint8), np.full((k // 128, 64), ka["scale"]), np.full((k // 128, 64), ka["zero"], np.uint8), 128)
    assert np.all(x @ w == ka["expected"])
    # The restated AVX CPU GEMV on packed tiles reaches the same exact value in bf16.
    s_bits = oracle.bf16_bits(np.full((k // 128, 64), ka["scale"], np.float32))
    packed = oracle.pack_tiles(np.full((k, 64), ka["q"], np.uint8), s_bits, np.full((k // 128, 64), ka["zero"], np.uint8))
    x_bits = oracle.bf16_bits(np.full(k, ka["x"], np.float32))
    for use_avx in (0, 1):
        y, _ = oracle.cpu_gemv_packed(x_bits, packed, k, 64, threads=2, use_avx=use_avx)
        assert np.all(oracle.bf16_bits_to_f32(y) == ka["expected"])


def test_zero_weights_give_zero(oracle):
    rng = np.random.default_rng(6)
    q = np.full((256, 128), 7, np.uint8)
    z = np.full((2, 128), 7, np.uint8)
    s = rng.uniform(0.01, 0.1, (2, 128))
    x = rng.standard_normal((3, 256))
    assert np.all(x @ oracle.dequantize(q, s, z, 128) == 0)


def test_brute_force_matches_vectorized(oracle):
    # Tiny shapes in pure-Python loops against the vectorized dequantize + matmul, g = 64.
    rng = np.random.default_rng(8)
    k, n, g = 128, 16, 64
    q, s_bits, z = oracle.random_weights(rng, k, n, g, "fp16")
    s = oracle.from_bits(s_bits, "fp16")
    x = rng.standard_normal(k)
    ref = x @ oracle.weights_f64(q, s_bits, z, g, "fp16")
    for col in range(n):
        acc = 0.0
        for kk in range(k):
            acc += x[kk] * (int(q[kk, col]) - int(z[kk // g, col])) * float(s[kk // g, col])
        assert abs(acc - ref[col]) <= 1e-9 * max(1.0, abs(ref[col]))


def test_cpu_gemv_restatement_vs_fp64(oracle):
    ka = GOLDEN["cpu_gemv_tolerance"]
    rng = np.random.default_rng(9)
    k, n = 1024, 640
    q, s, z = oracle.random_weights(rng, k, n, 128, "bf16", 0.002, 0.02, 0, 16)
    packed = oracle.pack_tiles(q, s, z)
    x_bits = oracle.bf16_bits((rng.standard_normal(k) * 0.5).astype(np.float32))
    ref = oracle.bf16_bits_to_f32(x_bits).astype(np.float64) @ oracle.weights_f64(q, s, z, 128, "bf16")
    outs = []
    for use_avx in (0, 1):
        y, branch = oracle.cpu_gemv_packed(x_bits, packed, k, n, threads=3, use_avx=use_avx)
        assert branch == (use_avx and oracle.cpu_has_avx512())
        got = oracle.bf16_bits_to_f32(y)
        np.testing.assert_allclose(got, ref, rtol=ka["rtol"], atol=ka["atol"])
        assert oracle.errors(got, ref)["rel_l2"] < 5e-3
        outs.append(got)
    # start/end columns select 64-column tiles and write absolute columns, like the reference.
    y, _ = oracle.cpu_gemv_packed(x_bits, packed, k, n, threads=2, start_col=128, end_col=320)
    got = oracle.bf16_bits_to_f32(y)
    np.testing.assert_array_equal(got[128:320], outs[1][128:320] if oracle.cpu_has_avx512() else outs[0][128:320])
    assert np.all(got[:128] == 0) and np.all(got[320:] == 0)


def test_cpu_ffn_decode_vs_oracle(oracle):
    rng = np.random.default_rng(10)
    h, inter = 256, 512
    gate = oracle.random_weights(rng, h, inter, 128, "bf16")
    up = oracle.random_weights(rng, h, inter, 128, "bf16")
    down = oracle.random_weights(rng, inter, h, 128, "bf16")
    tiles = [oracle.pack_tiles(*w) for w in (gate, up, down)]
    x_bits = oracle.bf16_bits(rng.standard_normal(h).astype(np.float32))
    y, _ = oracle.cpu_ffn_decode(x_bits, *tiles, h, inter, threads=2)
    ref, _ = oracle.ffn(oracle.bf16_bits_to_f32(x_bits)[None, :], gate, up, down, 128, "bf16")
    e = oracle.errors(oracle.bf16_bits_to_f32(y), ref[0])
    assert e["max_rel"] < 2e-2 and e["rel_l2"] < 1e-2, e


def test_ffn_split_invariant(oracle):
    # Y_G + Y_N == unsplit (reference.py:200-221; check_packing.py:119-124); endpoints equal the full FFN.
    rng = np.random.default_rng(11)
    h, inter, g = 256, 768, 64
    gate = oracle.random_weights(rng, h, inter, g, "fp16")
    up = oracle.random_weights(rng, h, inter, g, "fp16")
    down = oracle.random_weights(rng, inter, h, g, "fp16")
    x = oracle.round_to(rng.standard_normal((3, h)).astype(np.float32), "fp16")
    full, _ = oracle.ffn(x, gate, up, down, g, "fp16", round_act=False)
    for s in (0, 128, 384, 640, 768):
        parts = [oracle.ffn(x, gate, up, down, g, "fp16", round_act=False, channels=c)[0] for c in ((0, s), (s, inter)) if c[0] < c[1]]
        np.testing.assert_allclose(sum(parts), full, rtol=1e-10, atol=1e-10)


def test_partition_from_ratio_known_answers(oracle):
    ka = GOLDEN["partition_from_ratio"]
    for inter, ratio, align, exp in ka["cases"]:
        assert oracle.partition_from_ratio(inter, ratio, align) == exp
    for r in ka["rejected_ratios"]:
        with pytest.raises(ValueError):
            oracle.partition_from_ratio(32, _f(r), 4)


def test_rmsnorm_closed_form(oracle):
    x = np.array([[3.0, 4.0, 0.0, 0.0]])
    w = np.array([1.0, 2.0, 1.0, 1.0])
    got = oracle.rmsnorm(x, w, 0.0)
    np.testing.assert_allclose(got, [[3 / 2.5, 8 / 2.5, 0, 0]], rtol=1e-15)


def test_rmsnorm_eps_inside_the_root(oracle):
    # A row of equal values a: mean(x^2) = a^2, so normed = a / sqrt(a^2 + eps) * w exactly (rmsnorm.cu:48 adds eps
    # under the square root). At |a| = 1e-3 with eps = 1e-5 that is 0.30151..., far from a / (|a| + eps) = 0.990...
    # (eps outside the root) and from 1 (eps dropped).
    a, eps = 1e-3, 1e-5
    x = np.full((2, 64), a)
    x[1] *= -1
    w = np.linspace(0.5, 1.5, 64)
    got = oracle.rmsnorm(x, w, eps)
    exp = a / math.sqrt(a * a + eps)
    np.testing.assert_allclose(got[0], exp * w, rtol=1e-14)
    np.testing.assert_allclose(got[1], -exp * w, rtol=1e-14)
    assert abs(exp - 0.30151134457776363) < 1e-15


# ---- direct rounding from float64 ---------------------------------------------------------------------

def test_f16_from_f64_matches_numpy_direct_cast(oracle):
    # numpy converts float64 -> float16 directly from the double's bits (round to nearest even); values within a
    # float32 ulp of a float16 tie separate a direct rounding from one through float32.
    rng = np.random.default_rng(21)
    x = rng.standard_normal(20000) * np.exp(rng.uniform(-25, 12, 20000))
    ties = np.float16(rng.standard_normal(3000)).astype(np.float64)
    ulp = np.spacing(np.abs(ties.astype(np.float16))).astype(np.float64)
    near = np.concatenate([ties + ulp / 2, ties - ulp / 2, ties + ulp / 2 * (1 + 2.0 ** -40), ties + ulp / 2 * (1 - 2.0 ** -40)])
    vals = np.concatenate([x, near, [0.0, -0.0, 65519.99, 65520.0, 1e-8, -6e-8, 2.0 ** -25, 3 * 2.0 ** -26]])
    got = np.array([oracle.f64_to_bits(v, "fp16") for v in vals], np.uint16)
    with np.errstate(over="ignore"):  # 65520 rounds to infinity, as intended
        np.testing.assert_array_equal(got, vals.astype(np.float16).view(np.uint16))


def test_bf16_from_f64_ties(oracle):
    # 1 + 2^-8 is a bf16 tie (rounds to even: 1.0); 2^-40 above it must round up, which a detour through float32
    # (where 1 + 2^-8 + 2^-40 becomes the tie itself) would not do.
    assert oracle.f64_to_bits(1 + 2.0 ** -8, "bf16") == 0x3F80
    assert oracle.f64_to_bits(1 + 2.0 ** -8 + 2.0 ** -40, "bf16") == 0x3F81
    assert oracle.f64_to_bits(1 + 3 * 2.0 ** -8, "bf16") == 0x3F82  # tie between 0x3F81 and 0x3F82: even
    assert oracle.f64_to_bits(-3.0234375, "bf16") == 0xC042  # -(3 + 3/128): tie, even mantissa 3.03125
    rng = np.random.default_rng(22)
    v = (rng.standard_normal(5000) * np.exp(rng.uniform(-20, 20, 5000))).astype(np.float32)
    got = np.array([oracle.f64_to_bits(float(t), "bf16") for t in v], np.uint16)
    np.testing.assert_array_equal(got, oracle.bf16_bits(v))  # float32-exact inputs: one rounding either way


# ---- float64 FFN block (C) -----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,group", [("fp16", 128), ("bf16", 64), ("fp16", 32)])
def test_ffn_block_f64_matches_numpy(oracle, dtype, group):
    # The C block against the numpy formulation (dense dequantized matrices, matrix products): the float64 sums
    # agree to rounding, the rounded activations and outputs bit for bit.
    rng = np.random.default_rng(31)
    h, inter = 256, 384
    gate = oracle.random_weights(rng, h, inter, group, dtype)
    up = oracle.random_weights(rng, h, inter, group, dtype)
    down = oracle.random_weights(rng, inter, h, group, dtype)
    x_bits = oracle.to_bits((rng.standard_normal(h) * 3).astype(np.float32), dtype)
    w_bits = oracle.to_bits(rng.uniform(0.5, 1.5, h).astype(np.float32), dtype)
    eps = 1e-5
    out = oracle.ffn_block_f64(x_bits, w_bits, eps, gate, up, down, group, dtype, threads=2)
    x = oracle.from_bits(x_bits, dtype).astype(np.float64)
    normed = oracle.rmsnorm(x[None], oracle.from_bits(w_bits, dtype), eps)[0]
    normed_bits = np.array([oracle.f64_to_bits(v, dtype) for v in normed], np.uint16)
    np.testing.assert_array_equal(out["normed"], normed_bits)
    xn = oracle.from_bits(normed_bits, dtype).astype(np.float64)
    g = xn @ oracle.weights_f64(*gate, group, dtype)
    u = xn @ oracle.weights_f64(*up, group, dtype)
    np.testing.assert_allclose(out["g"], g, rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(out["u"], u, rtol=1e-11, atol=1e-11)
    act_bits = np.array([oracle.f64_to_bits(v, dtype) for v in oracle.silu(out["g"]) * out["u"]], np.uint16)
    np.testing.assert_array_equal(out["act"], act_bits)
    y = oracle.from_bits(act_bits, dtype).astype(np.float64) @ oracle.weights_f64(*down, group, dtype)
    np.testing.assert_allclose(out["y_raw"], y, rtol=1e-11, atol=1e-9)
    y_bits = np.array([oracle.f64_to_bits(v, dtype) for v in out["y_raw"]], np.uint16)
    np.testing.assert_array_equal(out["y"], y_bits)
    x_out = np.array([oracle.f64_to_bits(a + b, dtype) for a, b in zip(x, oracle.from_bits(y_bits, dtype))], np.uint16)
    np.testing.assert_array_equal(out["x_out"], x_out)
    # no norm: the block is the plain FFN of x plus the residual
    plain = oracle.ffn_block_f64(x_bits, None, eps, gate, up, down, group, dtype, threads=2)
    ref, _ = oracle.ffn(x[None], gate, up, down, group, dtype)
    np.testing.assert_allclose(plain["y_raw"], ref[0], rtol=1e-9, atol=1e-9)


def test_planted_ffn_block_gate_up_swap(oracle):
    # SiLU(g) u is not symmetric: a block with gate and up exchanged must differ.
    rng = np.random.default_rng(32)
    h, inter = 128, 256
    gate, up, down = (oracle.random_weights(rng, *s, 128, "fp16") for s in ((h, inter), (h, inter), (inter, h)))
    x_bits = oracle.to_bits(rng.standard_normal(h).astype(np.float32), "fp16")
    a = oracle.ffn_block_f64(x_bits, None, 0.0, gate, up, down, 128, "fp16", threads=1)
    b = oracle.ffn_block_f64(x_bits, None, 0.0, up, gate, down, 128, "fp16", threads=1)
    assert not np.array_equal(a["y"], b["y"])


# ---- rounding points of the reference's GPU kernels -------------------------------------------------------

def _bf16(v):
    return int(np.asarray([v], np.float32).view(np.uint32)[0] >> 16)


def test_hm_gemv_emul_constant_case(oracle):
    # docs/progress.md:457-460: x = 1/16, q = 9, z = 8, s = 1/16, K = 2048 gives exactly 8 (every partial sum is exact).
    k, n = 2048, 64
    x = np.full(k, _bf16(1 / 16), np.uint16)
    q = np.full((k, n), 9, np.uint8)
    s = np.full((k // 128, n), _bf16(1 / 16), np.uint16)
    z = np.full((k // 128, n), 8, np.uint8)
    y = oracle.hm_gemv_emul(x, q, s, z, threads=2)
    assert np.all(oracle.bf16_bits_to_f32(y) == 8.0)


def test_hm_gemv_emul_fp16_accumulation_known_answer(oracle):
    # Lane b = 0 of the reference GEMV takes rows sr * 8 (sr = 0..15) of each K tile into accumulator sr % 4. With
    # weights 1 (q = 9, z = 8, s = 1), x[0] = 1 and x = 2^-12 on the other rows 8 j, accumulator 0 holds 1 and each
    # further 2^-12 is below half an fp16 ulp of 1, so it stays 1; accumulators 1..3 each sum 32 x 2^-12 = 2^-7.
    # (a0 + a1) + (a2 + a3) = 1 + 2^-7 + 2^-6 = 1.0234375 (bf16-exact), where the exact sum 1 + 127 * 2^-12 rounds
    # to bf16 1.03125. A GEMV accumulating in fp32 gives 1.03125, one without per-lane accumulators another value.
    k, n = 1024, 64
    x = np.zeros(k, np.uint16)
    x[0::8] = _bf16(2.0 ** -12)
    x[0] = _bf16(1.0)
    q = np.full((k, n), 9, np.uint8)
    s = np.full((k // 128, n), _bf16(1.0), np.uint16)
    z = np.full((k // 128, n), 8, np.uint8)
    y = oracle.bf16_bits_to_f32(oracle.hm_gemv_emul(x, q, s, z, threads=2))
    assert np.all(y == np.float32(1.0234375)), y[:4]
    exact = 1 + 127 * 2.0 ** -12
    assert oracle.bf16_round(np.float32(exact)) == np.float32(1.03125)


def test_hm_gemv_emul_exact_regime_matches_float64(oracle):
    # Small integers keep every fp16 partial sum exact, so the emulation equals float64 rounded to bf16: this pins
    # the row, column and group indexing of the emulation.
    rng = np.random.default_rng(33)
    k, n = 512, 192
    xv = rng.integers(-1, 2, k).astype(np.float32)
    q = rng.integers(0, 16, (k, n), dtype=np.uint8)
    z = rng.integers(4, 12, (k // 128, n), dtype=np.uint8)
    s = np.full((k // 128, n), _bf16(1.0), np.uint16)
    y = oracle.hm_gemv_emul(oracle.bf16_bits(xv), q, s, z, threads=2)
    ref = xv.astype(np.float64) @ oracle.dequantize(q, np.ones((k // 128, n)), z, 128)
    np.testing.assert_array_equal(y, oracle.bf16_bits(ref.astype(np.float32)))


def test_hm_gemm_emul_rounds_each_weight_once_to_bf16(oracle):
    # (q - z) s = 3 * (1 + 2^-7) = 3.0234375 needs 9 significant bits: the reference GEMM stores it as bf16, a tie
    # that rounds to even (3.03125). With x = 1 on one row the output is that weight; the exact product is not.
    k, n = 128, 64
    x = np.zeros((2, k), np.uint16)
    x[0, 5] = _bf16(1.0)
    x[1] = _bf16(1 / 16)
    q = np.full((k, n), 11, np.uint8)
    z = np.full((1, n), 8, np.uint8)
    s = np.full((1, n), _bf16(1 + 2.0 ** -7), np.uint16)
    out = oracle.hm_gemm_emul(x, q, s, z, 128, threads=2)
    assert np.all(out[0] == np.float32(3.03125))
    assert np.all(out[1] == np.float32(3.03125 * 128 / 16))


def test_hm_gemm_emul_exact_regime_matches_float64(oracle):
    rng = np.random.default_rng(34)
    m, k, n, g = 3, 256, 128, 64
    xv = rng.integers(-2, 3, (m, k)).astype(np.float32)
    q = rng.integers(0, 16, (k, n), dtype=np.uint8)
    z = rng.integers(0, 16, (k // g, n), dtype=np.uint8)
    s = np.full((k // g, n), _bf16(0.5), np.uint16)
    out = oracle.hm_gemm_emul(oracle.bf16_bits(xv), q, s, z, g, threads=2)
    ref = xv.astype(np.float64) @ oracle.dequantize(q, np.full((k // g, n), 0.5), z, g)
    np.testing.assert_array_equal(out, ref.astype(np.float32))


def test_cpu_baseline_llama32_1b_shape(oracle):
    # Benchmark config 1: the restated reference AVX CPU path at the Llama-3.2-1B shape (H = 2048, I = 8192, g = 128,
    # bf16). Each GEMV as the reference checks it (test_layout_cpu.cpp:128-139: x = rand * 0.1, torch.allclose with
    # rtol 0.01, atol 0.1 against a dense matmul), then the whole decode FFN (gate, up, silu_ and mul_ in bf16,
    # down) against the float64 oracle by relative error.
    rng = np.random.default_rng(35)
    h, inter = 2048, 8192
    gate, up, down = (oracle.random_weights(rng, *s, 128, "bf16") for s in ((h, inter), (h, inter), (inter, h)))
    tiles = [oracle.pack_tiles(*w) for w in (gate, up, down)]
    for w, t, (k, n) in ((gate, tiles[0], (h, inter)), (down, tiles[2], (inter, h))):
        xb = oracle.to_bits((rng.uniform(0, 1, k) * 0.1).astype(np.float32), "bf16")
        y, _ = oracle.cpu_gemv_packed(xb, t, k, n, threads=4)
        ref = oracle.bf16_bits_to_f32(xb).astype(np.float64) @ oracle.weights_f64(*w, 128, "bf16")
        np.testing.assert_allclose(oracle.bf16_bits_to_f32(y), ref, rtol=0.01, atol=0.1)
    x_bits = oracle.to_bits(rng.standard_normal(h).astype(np.float32), "bf16")
    y, branch = oracle.cpu_ffn_decode(x_bits, *tiles, h, inter, threads=4)
    ref, _ = oracle.ffn(oracle.bf16_bits_to_f32(x_bits)[None, :].astype(np.float64), gate, up, down, 128, "bf16")
    e = oracle.errors(oracle.bf16_bits_to_f32(y), ref[0])
    print(f"config 1 CPU FFN decode ({'AVX-512' if branch else 'scalar'}): {e}")
    assert e["max_rel"] < 2e-2 and e["rel_l2"] < 1e-2, e
