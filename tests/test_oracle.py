"""CPU checks that pin the oracle (test infrastructure) before anything is compared against it.

Sources of truth, in order: the reference's own known-answer tests (crates/agens-core/src/reference.rs:123-156),
the layout definition in kernels/src/w4_gemv.cu:13-31 worked out by hand into literal words, the reference gates'
invariants (kernels/bench/test_wq.cu: W2 / W3 == W4 on the same values, range refusal; test_w4.cu: the fp64 bound),
and exact arithmetic (fp64 sums of at most 128 short products are exact).
"""
import ctypes

import numpy as np
import pytest

from _lib import (oracle, ptr, gen_container, gen_scales, gen_x, XorShift, f2bf_array, bf2f_array, ora_repack,
                  ora_fast, ora_exact, ora_ref_f32, ora_ref_f64, max_rel, max_rel_excess, max_ulp_bound)


def test_pack_known_answer():
    # reference.rs:124-130: q = -8..7 packs to 0x76543210 / 0xFEDCBA98 and round-trips
    O = oracle()
    q = np.arange(16, dtype=np.int8) - 8
    p = np.zeros(2, dtype=np.uint32)
    assert O.ora_pack_row(ptr(q), 16, ptr(p)) == 0
    assert int(p[0]) == 0x76543210 and int(p[1]) == 0xFEDCBA98
    back = np.zeros(16, dtype=np.int8)
    O.ora_unpack_row(ptr(p), 16, ptr(back))
    assert (back == q).all()
    bad = np.array([8, 0, 0, 0, 0, 0, 0, 0], dtype=np.int8)
    assert O.ora_pack_row(ptr(bad), 8, ptr(p)) == -1


def test_bf16_round_to_nearest_even():
    O = oracle()
    assert O.ora_f2bf(1.0) == 0x3F80
    assert O.ora_f2bf(-2.0) == 0xC000
    # 1 + 2^-8 is a tie between 1.0 and 1 + 2^-7: even mantissa (1.0) wins; 1 + 3*2^-8 rounds up to 1 + 2^-6
    assert O.ora_f2bf(1.0 + 2 ** -8) == 0x3F80
    assert O.ora_f2bf(1.0 + 3 * 2 ** -8) == 0x3F82
    assert abs(O.ora_bf2f(0x3FC0) - 1.5) == 0


def _quantized_case():
    # reference.rs:132-140: a deterministic 3 x 256 weight, quantised per 128-group, and a deterministic x
    out, inp = 3, 256
    i = np.arange(out * inp)
    w = (((i * 37) % 101).astype(np.float32) - 50.0) / 100.0
    j = np.arange(inp)
    x = f2bf_array((((j * 13) % 17).astype(np.float32) - 8.0) / 8.0)
    O = oracle()
    packed = np.zeros(out * inp // 8, dtype=np.uint32)
    scales = np.zeros(out * inp // 128, dtype=np.uint16)
    deq = np.zeros(out * inp, dtype=np.float32)
    for o in range(out):
        q = np.zeros(inp, dtype=np.int8)
        s = np.zeros(inp // 128, dtype=np.uint16)
        row = np.ascontiguousarray(w[o * inp:(o + 1) * inp])
        O.ora_quantize_row(ptr(row), inp, ptr(q), ptr(s))
        assert O.ora_pack_row(ptr(q), inp, ptr(packed[o * inp // 8:])) == 0
        scales[o * 2:(o + 1) * 2] = s
        deq[o * inp:(o + 1) * inp] = q.astype(np.float32) * bf2f_array(s)[np.arange(inp) // 128]
    return out, inp, w, x, packed, scales, deq


def test_gemv_matches_dequant_reference_case():
    # reference.rs:141-148: |y - sum x * deq| < 1e-3 (1 + |r|)
    out, inp, w, x, packed, scales, deq = _quantized_case()
    y = ora_ref_f32(x, 1, packed, scales, out, inp, 128)[0]
    xf = bf2f_array(x).astype(np.float32)
    for o in range(out):
        r = float(np.sum(xf * deq[o * inp:(o + 1) * inp], dtype=np.float32))
        assert abs(y[o] - r) < 1e-3 * (1.0 + abs(r))


def test_dequant_known_answer_and_g64_repeat():
    # reference.rs:149-155: dequant == bf16(q * s) bitwise; a g64 container with repeated scales dequantises the same
    out, inp, w, x, packed, scales, deq = _quantized_case()
    for bits in (4,):
        rc, wt, st = ora_repack(bits, packed, scales, out, inp, 128)
        assert rc == 0
        d = np.zeros(out * inp, dtype=np.uint16)
        assert oracle().ora_dequant_kt_rows(bits, ptr(wt), ptr(st), ptr(d), out, inp, 128, 0, out) == 0
        assert (d == f2bf_array(deq)).all()
        s64 = np.repeat(scales, 2)
        rc, wt64, st64 = ora_repack(bits, packed, s64, out, inp, 64)
        d64 = np.zeros_like(d)
        assert oracle().ora_dequant_kt_rows(bits, ptr(wt64), ptr(st64), ptr(d64), out, inp, 64, 0, out) == 0
        assert (d64 == d).all()


def _chunk(bits, wt, rec, lane):
    out = np.zeros(4, dtype=np.uint32)
    oracle().ora_kt_chunk(bits, ptr(wt), rec, lane, ptr(out))
    return out


def test_kt_layout_literal_words():
    # w4_gemv.cu:13-31 worked by hand: input v of every lane chunk holds q = (v % 2^bits) - 2^(bits-1).
    # W3: 2-bit fields 0,1,2,3,0,1,2,3,... -> byte 0xE4 (0 | 1<<2 | 2<<4 | 3<<6); third bits 0,0,0,0,1,1,1,1 -> 0xF0.
    # W2: fields 0,1,2,3 repeating -> 0xE4 bytes.
    n, k = 2, 1024
    for bits, lo_word, hi_word in ((3, 0xE4E4E4E4, 0xF0F0F0F0), (2, 0xE4E4E4E4, None)):
        span = 1 << bits
        q = ((np.arange(k) % span) - span // 2).astype(np.int8)
        # a period-8 (W3) / period-4 (W2) pattern: within each 32-input chunk input v has value v % span
        packed = np.zeros(n * k // 8, dtype=np.uint32)
        for o in range(n):
            assert oracle().ora_pack_row(ptr(q), k, ptr(packed[o * k // 8:])) == 0
        scales = np.arange(n * k // 128, dtype=np.uint16) + 0x3F80
        rc, wt, st = ora_repack(bits, packed, scales, n, k, 128)
        assert rc == 0
        words = wt.view(np.uint32)
        rec_words = 32 * bits
        for rec in range(n):
            r = words[rec * rec_words:(rec + 1) * rec_words]
            assert (r[:64] == lo_word).all()
            if hi_word is not None:
                assert (r[64:96] == hi_word).all()
        # scales: record (t, o) slot i = container scale of row o, group 8t + i
        assert (st.reshape(n, 8) == scales.reshape(n, 8)).all()
    # W4: record (t, o) lane chunk l = container chunk 32t + l of row o, byte for byte
    n, k = 3, 2048
    packed = XorShift(12345).words(n * k // 8)
    scales = np.arange(n * k // 128, dtype=np.uint16)
    rc, wt, st = ora_repack(4, packed, scales, n, k, 128)
    c = wt.view(np.uint32).reshape(k // 1024, n, 32, 4)
    cont = packed.reshape(n, k // 32, 4)
    for t in range(k // 1024):
        assert (c[t] == cont[:, 32 * t:32 * t + 32, :]).all()
        assert (st.reshape(k // 1024, n, 8)[t] == scales.reshape(n, k // 128)[:, 8 * t:8 * t + 8]).all()


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("group", [64, 128])
def test_wq_chunks_equal_w4_chunks(bits, group):
    # test_wq.cu:1-17: a W{bits} KT chunk read back is the W4 KT chunk of the same values (ragged n, padded k)
    n, k = 77, 1152
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(7 + bits, n, k, lo, span)
    scales = gen_scales(9, n * k // group)
    rc4, wt4, st4 = ora_repack(4, packed, scales, n, k, group)
    rcb, wtb, stb = ora_repack(bits, packed, scales, n, k, group)
    assert rc4 == 0 and rcb == 0 and (st4 == stb).all()
    tiles = (k + 1023) // 1024
    for rec in range(0, tiles * n, 5):
        for lane in range(32):
            assert (_chunk(4, wt4, rec, lane) == _chunk(bits, wtb, rec, lane)).all()


def test_repack_range_check():
    # test_wq.cu:249-269: W2 refuses a 3-bit value, W3 a 4-bit value, W3 accepts W2 values and the extremes
    n, k = 64, 1024
    w3vals = gen_container(1, n, k, -4, 8)
    w4vals = gen_container(2, n, k, -8, 16)
    w2vals = gen_container(3, n, k, -2, 4)
    s = gen_scales(4, n * k // 64)
    assert ora_repack(2, w3vals, s, n, k, 64)[0] == 1
    assert ora_repack(3, w4vals, s, n, k, 64)[0] == 1
    assert ora_repack(3, w2vals, s, n, k, 64)[0] == 0
    ext = np.full(n * k // 8, 0x4B4B4B4B, dtype=np.uint32)  # nibbles 0xB (q=3) and 0x4 (q=-4)
    assert ora_repack(3, ext, s, n, k, 64)[0] == 0
    assert oracle().ora_repack_kt(4, ptr(w4vals), ptr(s), ptr(np.zeros(1, np.uint8)), ptr(np.zeros(1, np.uint16)),
                                  n, 1000, 128) == 1  # k % group != 0


def _sample(seed, n, k, group, m, lo=-8, span=16, xs=1.0):
    packed = gen_container(seed, n, k, lo, span)
    scales = gen_scales(seed + 1, n * k // group)
    x = gen_x(seed + 2, m * k, xs)
    return packed, scales, x


def test_fast_group_sums_are_exact():
    # the integer group sum times 2^(E-148) equals the exact (fp64) sum of x * q when no input is below 2^-14 of
    # the group's largest; with tiny inputs mixed in it differs by less than one unit 2^(E-148) per input
    n, k, group = 8, 2048, 128
    packed, scales, x = _sample(11, n, k, group, 1)
    rc, wt, st = ora_repack(4, packed, scales, n, k, group)
    q = np.zeros(n * k, dtype=np.int8)
    for o in range(n):
        oracle().ora_unpack_row(ptr(packed[o * k // 8:]), k, ptr(q[o * k:]))
    xf = bf2f_array(x).astype(np.float64)
    E = ctypes.c_int()
    for o in range(n):
        for g in range(k // group):
            gs = oracle().ora_fast_group_sum(4, ptr(x), ptr(wt), n, k, group, o, g, ctypes.byref(E))
            sl = slice(g * group, (g + 1) * group)
            exact = float(np.sum(xf[sl] * q[o * k:(o + 1) * k][sl].astype(np.float64)))
            got = np.ldexp(float(gs), E.value - 148)
            small = np.abs(xf[sl]) < np.ldexp(1.0, E.value - 127 - 14)
            if not small.any():
                assert got == exact
            else:
                assert abs(got - exact) <= 8 * small.sum() * np.ldexp(1.0, E.value - 148)


@pytest.mark.parametrize("bits,group,n,k", [(4, 128, 256, 5120), (3, 128, 128, 2048), (2, 64, 96, 3072),
                                            (4, 64, 64, 1152), (3, 128, 77, 640)])
def test_fast_and_exact_within_reference_bounds(bits, group, n, k):
    # BASELINE tolerance (max rel err <= 2e-3 vs the fp32-accumulated reference, measured as bench_gemv.cu:146-148,
    # beyond the bf16 output rounding every bf16 output carries) and the reference gate's bound vs fp64
    # (test_w4.cu:123-141), for both numerics
    if k % group:
        pytest.skip("k % group")
    lo, span = -(1 << (bits - 1)), 1 << bits
    m = 3
    packed, scales, x = _sample(20 + bits, n, k, group, m, lo, span)
    rc, wt, st = ora_repack(bits, packed, scales, n, k, group)
    assert rc == 0
    ref32 = ora_ref_f32(x, m, packed, scales, n, k, group)
    ref64, mag = ora_ref_f64(x, m, packed, scales, n, k, group)
    yf = ora_fast(bits, x, m, wt, st, n, k, group)
    ye = ora_exact(bits, x, m, wt, st, n, k, group)
    assert max_rel_excess(yf, ref32) <= 2e-3
    assert max_rel_excess(ye, ref32) <= 2e-3
    # the raw measure is bounded by the output rounding alone (2^-8 relative) plus the tiny accumulation error
    assert max_rel(yf, ref32) <= 2 ** -8 + 2e-3
    assert max_ulp_bound(yf, ref64, mag) <= 1.0
    assert max_ulp_bound(ye, ref64, mag) <= 1.0


def test_exact_bf16w_against_rounded_weights():
    # bf16w = 1 (Marlin numerics): within the bound of fp64 over the bf16(q * s) weights (test_w4.cu section 5)
    n, k, group, m = 64, 2048, 128, 2
    packed, scales, x = _sample(31, n, k, group, m)
    rc, wt, st = ora_repack(4, packed, scales, n, k, group)
    d = np.zeros(n * k, dtype=np.uint16)
    assert oracle().ora_dequant_kt_rows(4, ptr(wt), ptr(st), ptr(d), n, k, group, 0, n) == 0
    wq = bf2f_array(d).astype(np.float64).reshape(n, k)
    xf = bf2f_array(x).astype(np.float64).reshape(m, k)
    ref = xf @ wq.T
    mag = np.abs(xf) @ np.abs(wq).T
    y = ora_exact(4, x, m, wt, st, n, k, group, bf16w=1)
    assert max_ulp_bound(y, ref, mag) <= 1.0


@pytest.mark.parametrize("bits", [2, 3])
def test_oracle_wq_equals_w4(bits):
    # test_wq.cu: every numerics gives the W4 bits on W{bits} weights of the same values
    n, k, group, m = 50, 3072, 128, 2
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed, scales, x = _sample(40 + bits, n, k, group, m, lo, span)
    _, wt4, st4 = ora_repack(4, packed, scales, n, k, group)
    _, wtb, stb = ora_repack(bits, packed, scales, n, k, group)
    assert (ora_fast(4, x, m, wt4, st4, n, k, group) == ora_fast(bits, x, m, wtb, stb, n, k, group)).all()
    assert (ora_exact(4, x, m, wt4, st4, n, k, group) == ora_exact(bits, x, m, wtb, stb, n, k, group)).all()


# ------------------------------------------------------------------------------------------------ INT8 LM head GEMV
def ora_i8(x, q, scale, m, n, k, ldy=None):
    ldy = ldy or n
    y = np.zeros(m * ldy, dtype=np.uint16)
    oracle().ora_i8_gemv(ptr(x), ptr(q), ptr(scale), ptr(y), m, n, k, ldy)
    return y


def test_i8_gemv_exact_integer_products():
    """Small-integer activations: every product and partial sum is an exact fp32 integer, so any summation order gives
    the exact dot product; y = bf16(fp32(S) * scale) pins the indexing (chunks, inputs, tokens, rows)."""
    rng = np.random.default_rng(5)
    m, n, k = 3, 9, 16 * 65  # 65 chunks: lanes 0 gets three, others two
    xi = rng.integers(-4, 5, size=(m, k))
    q = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
    scale = (rng.random(n) * 0.01 + 1e-3).astype(np.float32)
    x = f2bf_array(xi.astype(np.float32).ravel())
    y = ora_i8(x, q, scale, m, n, k).reshape(m, n)
    S = xi.astype(np.int64) @ q.astype(np.int64).T  # exact
    want = f2bf_array((S.astype(np.float32) * scale[None, :]).ravel()).reshape(m, n)
    assert np.array_equal(y, want)


def test_i8_gemv_summation_order_known_answers():
    """Hand-computed values where the reference's order (i8_gemv.cu:44-70) differs from a plain left-to-right sum:
    lane l's partial takes chunks l, l + 32, ..., each chunk's fma chain starts from 0, and the 32 partials meet in an
    xor butterfly.  k = 64 chunks, q = 1 where x is set, scale 1."""
    k, n, m = 16 * 64, 1, 1
    q = np.ones((n, k), dtype=np.int8)
    scale = np.ones(n, dtype=np.float32)

    def run(vals):
        xf = np.zeros(k, dtype=np.float32)
        for i, v in vals.items():
            xf[i] = v
        return bf2f_array(ora_i8(f2bf_array(xf), q, scale, m, n, k))[0]

    # chunks 0 (lane 0): 2^24, 1 (lane 1): 1, 2 (lane 2): -2^24, 3 (lane 3): 1.  Butterfly distance 2 pairs lanes
    # 0 + 2 = 0 and 1 + 3 = 2, distance 1 gives 2; left to right gives ((2^24 + 1) - 2^24) + 1 = 1
    assert run({0: 2.0 ** 24, 16: 1.0, 32: -(2.0 ** 24), 48: 1.0}) == 2.0
    # lane 0: chunk 0 = 2^24, chunk 32 = 1 + 1 (its own chain from 0: 2) -> 2^24 + 2; lane 2: chunk 2 = -2^24.
    # Result 2; one fma chain carried across chunks would give 2^24 + 1 + 1 = 2^24 and then 0
    assert run({0: 2.0 ** 24, 16 * 32: 1.0, 16 * 32 + 1: 1.0, 32: -(2.0 ** 24)}) == 2.0
    # within a chunk the chain is sequential: 2^24, 1, -2^24 in inputs 0..2 of chunk 0: fma(1, 1, 2^24) = 2^24,
    # then 0 (a pairwise sum of the chunk would keep the 1)
    assert run({0: 2.0 ** 24, 1: 1.0, 2: -(2.0 ** 24)}) == 0.0


def test_i8_gemv_within_fp64_bound():
    rng = np.random.default_rng(7)
    m, n, k = 2, 33, 5120
    x = f2bf_array(rng.standard_normal(m * k).astype(np.float32))
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    scale = (rng.random(n) * 0.02 + 1e-4).astype(np.float32)
    y = bf2f_array(ora_i8(x, q, scale, m, n, k)).reshape(m, n).astype(np.float64)
    xf = bf2f_array(x).reshape(m, k).astype(np.float64)
    ref = (xf @ q.astype(np.float64).T) * scale[None, :]
    mag = (np.abs(xf) @ np.abs(q.astype(np.float64)).T) * scale[None, :]
    # bf16 output rounding (2^-9 relative) plus fp32 summation error (k * 2^-24 of sum |x q|)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -8 + mag * k * 2.0 ** -24)


# ------------------------------------------------------------------------------------------------ exact path order
def exact_order_case(vals, k=4096):
    """One W4 row of q = 1 (container nibbles 9), scales 1.0, group 128; x zero but for `vals` {input: value}."""
    n = 1
    packed = np.full(n * k // 8, 0x99999999, dtype=np.uint32)
    scales = np.full(n * k // 128, 0x3F80, dtype=np.uint16)
    rc, wt, st = ora_repack(4, packed, scales, n, k, 128)
    assert rc == 0
    xf = np.zeros(k, dtype=np.float32)
    for i, v in vals.items():
        xf[i] = v
    return f2bf_array(xf), wt, st


# Hand-computed answers where the reference's exact order (w4_gemv.cu:117-127, 279-349: per lane chunk four 8-input fma
# chains from 0 added left to right, acc = fma(d, s, acc) over the lane's tiles in order, xor butterfly 16..1 over the
# 32 lanes) differs from other orders.  Input i: tile i // 1024, lane (i % 1024) // 32, chunk word (i % 32) // 8.
EXACT_ORDER_CASES = [
    # one 8-input chain: 2^24, +1 (lost), +1 (lost), -2^24 -> 0 (a pairwise sum gives 1)
    ({0: 2.0 ** 24, 1: 1.0, 2: 1.0, 3: -(2.0 ** 24)}, 0.0),
    # the chunk's four chains added left to right: ((2^24 + 1) + 1) - 2^24 = 0 (pairwise: 1)
    ({0: 2.0 ** 24, 8: 1.0, 16: 1.0, 24: -(2.0 ** 24)}, 0.0),
    # one lane over its tiles, acc = fma(d, s, acc) in tile order: 0 (pairwise over tiles: 1)
    ({0: 2.0 ** 24, 1024: 1.0, 2048: 1.0, 3072: -(2.0 ** 24)}, 0.0),
    # lanes 0..3 of one tile through the butterfly: (l0 + l2) + (l1 + l3) = 0 + 2 (left to right: 1)
    ({0: 2.0 ** 24, 32: 1.0, 64: -(2.0 ** 24), 96: 1.0}, 2.0),
]


@pytest.mark.parametrize("case", range(len(EXACT_ORDER_CASES)))
@pytest.mark.parametrize("bf16w", [0, 1])
def test_exact_order_known_answers(case, bf16w):
    vals, want = EXACT_ORDER_CASES[case]
    x, wt, st = exact_order_case(vals)
    y = ora_exact(4, x, 1, wt, st, 1, 4096, 128, bf16w=bf16w)
    assert bf2f_array(y.reshape(-1))[0] == want


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_fast_nonfinite_activations_like_fp32_path(bits):
    # The default numerics' definition for non-finite activations, pinned against the reference's fp32 path
    # (reference.rs:53-71, restated by ora_gemv_ref_f32): with one Inf per group every output is NaN / +Inf / -Inf
    # exactly where the fp32 path's is (an Inf times q = 0 is NaN there, S = 0 here; Infs of two groups with opposite
    # signs meet as Inf - Inf); a NaN input makes every output NaN; a token without non-finite inputs is unaffected.
    n, k, group = 64, 2048, 128
    lo, span = -(1 << (bits - 1)), 1 << bits
    packed = gen_container(61 + bits, n, k, lo, span)
    scales = gen_scales(62, n * k // group)
    rc, wt, st = ora_repack(bits, packed, scales, n, k, group)
    assert rc == 0
    m = 4
    x = gen_x(63, m * k).reshape(m, k)
    clean = x[3].copy()
    x[0, 130] = 0x7F80                      # +Inf in group 1
    x[1, 5], x[1, 2000] = 0xFF80, 0x7F80    # -Inf in group 0, +Inf in group 15
    x[2, 300] = 0x7FC0                      # NaN in group 2
    x = x.reshape(-1)
    y = bf2f_array(ora_fast(bits, x, m, wt, st, n, k, group))
    ref = ora_ref_f32(x, m, packed, scales, n, k, group)
    for t in (0, 1):
        assert np.array_equal(np.isnan(y[t]), np.isnan(ref[t]))
        assert np.array_equal(np.isposinf(y[t]), np.isposinf(ref[t]))
        assert np.array_equal(np.isneginf(y[t]), np.isneginf(ref[t]))
    # rows whose weight at the Inf input is 0 are NaN in both; the others +-Inf with the sign of q
    q = np.zeros(n * k, dtype=np.int8)
    for o in range(n):
        oracle().ora_unpack_row(ptr(packed[o * k // 8:]), k, ptr(q[o * k:]))
    q = q.reshape(n, k)
    assert np.array_equal(np.isnan(y[0]), q[:, 130] == 0)
    assert np.array_equal(np.isposinf(y[0]), q[:, 130] > 0)
    assert np.all(np.isnan(y[2]))
    one = bf2f_array(ora_fast(bits, clean, 1, wt, st, n, k, group))[0]
    assert np.array_equal(one, y[3])
