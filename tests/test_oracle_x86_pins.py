"""Pins for the oracle's x86 AVX2 restatements, which the reference's golden
vectors (generic arms only) do not cover.  Each case is built so that the
reference's specification gives one answer and a plausible mistake another.

quantize_row_q8_0, AVX2 arm (src/ggml/cpu/quants/x86/rows.zig:18-105):
  - ties round to even (`_mm256_round_ps(.., _MM_ROUND_NEAREST)`), where
    quantize_row_q8_0_ref rounds them away: on a block with amax = 127 the
    multiplier is exactly 1, so 2.5, 3.5, -2.5, 126.5, 0.5, -0.5 give 2, 4,
    -2, 126, 0, 0 (the ref gives 3, 4, -3, 127, 1, -1);
  - the multiplier is `127 / amax`, not `1 / d` with d = amax / 127 (the ref):
    blocks are searched (fixed seed) on which the two f32 multipliers round
    some x * id to different integers, and the restatement must give the
    127 / amax codes there;
  - d = amax / 127 stored as f16, the same field as the ref.

vec_dot AVX2 arms (x86/k.zig:256-343 q4_K, :454-552 q6_K; x86/legacy.zig:
537-572 q8_0): eight f32 lanes accumulate `acc = fma(d, float(sumi), acc)`
block after block, and hsum_float_8 (x86/common.zig:37-43) folds them as
((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)); q4_K adds its four min
lanes once at the end, folded as (m0 + m2) + (m1 + m3).  The cases place
+-2^25 and 1 in chosen lanes of chosen blocks (integer lane sums of +-1,
block scales 2^25 or 1, so every product is exact): under the reference's
order the 1 survives, while a sequential lane sum, a per-block horizontal
sum, another pairing in hsum_float_8, or mins folded into the lanes lose it
against 2^25 (ulp 4).  Each case also checks, in numpy f32 on the same lane
values, that the alternative it targets gives the other answer.
"""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.skipif(not O.has_avx2(), reason="host has no AVX2")

BIG = np.float32(2.0 ** 25)


def _f16(v):
    return np.float16(v).view(np.uint16)


# ---------------------------------------------------------------- quantize_row_q8_0 (AVX2)

def _q8_0_avx2(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    O.lib().orc_quantize_row_q8_0_avx2(x.ctypes.data, out.ctypes.data, x.size)
    return out.reshape(-1, 34)


def test_q8_0_avx2_rounds_ties_to_even():
    x = np.zeros(32, np.float32)
    x[:7] = [127.0, 2.5, 3.5, -2.5, 126.5, 0.5, -0.5]
    x[7:11] = [1.5, -1.5, 125.5, -126.5]
    avx = _q8_0_avx2(x)
    ref = O.quantize_ref(O.TYPE_Q8_0, x).reshape(-1, 34)
    codes = avx[0, 2:].view(np.int8)[:11].tolist()
    assert codes == [127, 2, 4, -2, 126, 0, 0, 2, -2, 126, -126]
    assert ref[0, 2:].view(np.int8)[:11].tolist() == [127, 3, 4, -3, 127, 1, -1, 2, -2, 126, -127]
    assert avx[0, :2].view(np.uint16)[0] == ref[0, :2].view(np.uint16)[0] == _f16(1.0)


def _codes(x, id_):
    return np.rint(x * id_).astype(np.int64)  # np.rint rounds half to even, as the AVX2 arm


def test_q8_0_avx2_multiplier_is_127_over_amax():
    """Find blocks where id = 127/amax and id = 1/(amax/127) (f32 both)
    quantize some element differently; the restatement follows 127/amax."""
    rng = np.random.default_rng(7)
    found = []
    while len(found) < 8:
        x = rng.standard_normal(32).astype(np.float32) * np.float32(rng.uniform(0.01, 10.0))
        amax = np.max(np.abs(x))
        id_avx = np.float32(127.0) / amax
        id_ref = np.float32(1.0) / (amax / np.float32(127.0))
        if id_avx == id_ref:
            continue
        a, r = _codes(x, id_avx), _codes(x, id_ref)
        if np.any(a != r):
            found.append((x, a, r))
    for x, want, other in found:
        got = _q8_0_avx2(x)[0, 2:].view(np.int8).astype(np.int64)
        np.testing.assert_array_equal(got, want)
        assert np.any(got != other)


def test_q8_0_avx2_matches_ref_away_from_ties():
    """Away from ties and multiplier differences the two arms agree exactly
    (same d, same codes): normal data quantized by both, the differing codes
    are only at x * id within 1e-3 of a half integer or where the two f32
    multipliers differ."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(32 * 512).astype(np.float32)
    avx = _q8_0_avx2(x)
    ref = O.quantize_ref(O.TYPE_Q8_0, x).reshape(-1, 34)
    np.testing.assert_array_equal(avx[:, :2], ref[:, :2])
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1, keepdims=True)
    id_avx = np.float32(127.0) / amax
    id_ref = np.float32(1.0) / (amax / np.float32(127.0))
    diff = avx[:, 2:].view(np.int8) != ref[:, 2:].view(np.int8)
    frac = np.abs(np.abs(xb * id_avx) % 1.0 - 0.5)
    assert np.all(diff <= ((frac < 1e-3) | (id_avx != id_ref)))
    np.testing.assert_array_equal(avx[:, 2:].view(np.int8), _codes(xb, id_avx))


# ---------------------------------------------------------------- block builders

def _q8_K(d, elems):
    """One Q8_K block {d f32, qs[256] i8, bsums[16] i16} with q8 values at the
    given elements and bsums consistent with them."""
    b = np.zeros(292, np.uint8)
    b[0:4] = np.array([d], np.float32).view(np.uint8)
    qs = np.zeros(256, np.int8)
    for e, v in elems.items():
        qs[e] = v
    b[4:260] = qs.view(np.uint8)
    b[260:292] = qs.astype(np.int16).reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    return b


def _q4_K(elems, d=1.0, dmin=0.0, sc=None, mins=None):
    """One Q4_K block with 4-bit codes at the given elements (others 0);
    sub-block scales / mins 0-3 from sc / mins (6-bit, stored plainly in
    scales[j] / scales[j + 4] as getScaleMinK4 reads them for j < 4)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([_f16(dmin)], np.uint16).view(np.uint8)
    for j, v in enumerate(sc or []):
        b[4 + j] = v
    for j, v in enumerate(mins or []):
        b[4 + 4 + j] = v
    for e, q in elems.items():
        c, r = divmod(e, 64)
        byte = 16 + 32 * c + (r % 32)
        b[byte] |= (q & 15) << (4 if r >= 32 else 0)
    return b


def _q6_K(elems, d=1.0, sc=None):
    """One Q6_K block {ql[128], qh[64], scales[16] i8, d f16} with 6-bit codes
    at the given elements (others 0), the layout of dequantize_row_q6_K."""
    b = np.zeros(210, np.uint8)
    for e, q in elems.items():
        n, r = divmod(e, 128)
        part, l = divmod(r, 32)
        ql = 64 * n + l + (32 if part in (1, 3) else 0)
        b[ql] |= (q & 15) << (4 if part >= 2 else 0)
        b[128 + 32 * n + l] |= ((q >> 4) & 3) << (2 * part)
    scales = np.zeros(16, np.int8)
    for j, v in enumerate(sc or []):
        scales[j] = v
    b[192:208] = scales.view(np.uint8)
    b[208:210] = np.array([_f16(d)], np.uint16).view(np.uint8)
    return b


def _q8_0(d, elems):
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    qs = np.zeros(32, np.int8)
    for e, v in elems.items():
        qs[e] = v
    b[2:] = qs.view(np.uint8)
    return b


# ---------------------------------------------------------------- accumulation-order cases
#
# A case is a list of blocks, each (scale, {lane: +-1}); lane l of block b
# then holds scale_b * sign exactly.  Expected: 1.0 under the reference.

CASES = {
    # a0 = 2^25, a4 = -2^25, a1 = 1: hsum pairs a0 with a4 first
    "hsum_upper_lower": ([(BIG, {0: 1, 4: -1}), (1.0, {1: 1})], "sequential"),
    # lane 0 cancels across blocks; a per-block horizontal sum loses the 1
    "lanes_across_blocks": ([(BIG, {0: 1}), (1.0, {1: 1}), (BIG, {0: -1})], "per_block"),
    # a0 = 2^25, a2 = 1, a4 = -2^25: (a0 + a4) before (a2 + a6)
    "hsum_pairs_0_4": ([(BIG, {0: 1, 4: -1}), (1.0, {2: 1})], "pair_0_2"),
    # a1 = 2^25, a3 = -2^25, a0 = 1: even and odd lanes are folded apart
    "hsum_even_odd": ([(BIG, {1: 1, 3: -1}), (1.0, {0: 1})], "even_odd_mixed"),
}


def _alt(kind, blocks):
    """The targeted alternative order, in numpy f32 on the same lane values."""
    f = np.float32
    lanes = np.zeros((len(blocks), 8), np.float32)
    for b, (s, ls) in enumerate(blocks):
        for l, v in ls.items():
            lanes[b, l] = f(s) * f(v)
    acc = lanes.sum(axis=0, dtype=np.float32) if len(blocks) else np.zeros(8, np.float32)
    if kind == "sequential":
        r = f(0)
        for v in acc:
            r = f(r + v)
        return r
    if kind == "per_block":
        r = f(0)
        for row in lanes:
            r = f(r + _hsum8(row))
        return r
    if kind == "pair_0_2":
        return f(f(f(acc[0] + acc[2]) + f(acc[4] + acc[6])) + f(f(acc[1] + acc[3]) + f(acc[5] + acc[7])))
    if kind == "even_odd_mixed":
        return f(f(f(acc[0] + acc[4]) + f(acc[1] + acc[5])) + f(f(acc[2] + acc[6]) + f(acc[3] + acc[7])))
    raise ValueError(kind)


def _hsum8(a):
    f = np.float32
    return f(f(f(a[0] + a[4]) + f(a[2] + a[6])) + f(f(a[1] + a[5]) + f(a[3] + a[7])))


@pytest.mark.parametrize("case", list(CASES))
def test_alternatives_lose_the_one(case):
    """The case design: the targeted alternative order gives 0, the
    reference's 1 (in numpy f32 on the constructed lane values)."""
    blocks, kind = CASES[case]
    assert _alt(kind, blocks) == 0.0


# q4_K: lane l of sumi takes low-nibble elements 64c + 4l .. 4l + 3 of sub-block 2c
# (x86/k.zig:317-333); element 4l of sub-block 0 (scale 1) puts q * q8 in lane l.
# q6_K: element e adds sc * q * q8 to lane (e % 32) // 4 and subtracts
# 32 * sc * q8 from lane e // 32 (the bsums term, x86/k.zig:487-549); e = 36 l
# keeps both in lane l, and q = 33 leaves sc * q8.
# q8_0: lane l is the sum of the products 4l .. 4l + 3 (mul_sum_i8_pairs_float).

def _dot_q4_K(blocks):
    xs, ys = [], []
    for s, ls in blocks:
        xs.append(_q4_K({4 * l: 1 for l in ls}, sc=[1]))
        ys.append(_q8_K(s, {4 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_Q4_K, O.IMPL_AVX2, 256 * len(blocks), np.concatenate(xs), np.concatenate(ys))


def _dot_q6_K(blocks):
    xs, ys = [], []
    for s, ls in blocks:
        xs.append(_q6_K({36 * l: 33 for l in ls}, sc=[1] * 16))
        ys.append(_q8_K(s, {36 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_Q6_K, O.IMPL_AVX2, 256 * len(blocks), np.concatenate(xs), np.concatenate(ys))


def _dot_q8_0(blocks):
    xs, ys = [], []
    for s, ls in blocks:
        # d = f16(x.d) * f16(y.d): 2^25 = 2^12 * 2^13, 1 = 1 * 1
        dx, dy = (4096.0, 8192.0) if s == BIG else (1.0, 1.0)
        xs.append(_q8_0(dx, {4 * l: 1 for l in ls}))
        ys.append(_q8_0(dy, {4 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_Q8_0, O.IMPL_AVX2, 32 * len(blocks), np.concatenate(xs), np.concatenate(ys))


def _q4_0(d, elems):
    """One Q4_0 block {d f16, qs[16]}: code 8 (weight 0) but at the given
    elements; element j < 16 is the low nibble of qs[j], j >= 16 the high
    nibble of qs[j - 16]."""
    codes = np.full(32, 8, np.int64)
    for e, q in elems.items():
        codes[e] = q
    b = np.zeros(18, np.uint8)
    b[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    b[2:] = (codes[:16] | (codes[16:] << 4)).astype(np.uint8)
    return b


def _q5_K(elems, d=1.0, dmin=0.0, sc=None, mins=None):
    """One Q5_K block {d, dmin f16, scales[12], qh[32], qs[128]}: 5-bit codes
    at the given elements (others 0); element 64c + r takes the low (r < 32)
    or high nibble of qs[32c + r % 32] and bit 2c (+1 for the high half) of
    qh[r % 32]."""
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([_f16(dmin)], np.uint16).view(np.uint8)
    for j, v in enumerate(sc or []):
        b[4 + j] = v
    for j, v in enumerate(mins or []):
        b[8 + j] = v
    for e, q in elems.items():
        c, r = divmod(e, 64)
        hi = r >= 32
        b[48 + 32 * c + r % 32] |= (q & 15) << (4 if hi else 0)
        b[16 + r % 32] |= ((q >> 4) & 1) << (2 * c + (1 if hi else 0))
    return b


def _iq4_xs(elems, d=1.0):
    """One IQ4_XS block {d f16, scales_h u16, scales_l[4], qs[128]}: group 0's
    scale ls = 33 (ls - 32 = 1), the given codes at group-0 elements (element
    j < 16 the low nibble of qs[j], 16..31 the high nibble of qs[j - 16]),
    code 8 (level 1) elsewhere."""
    b = np.zeros(136, np.uint8)
    b[0:2] = np.array([_f16(d)], np.uint16).view(np.uint8)
    b[2:4] = np.array([2], np.uint16).view(np.uint8)   # scales_h: group 0 high bits = 2
    b[4] = 1                                            # scales_l: group 0 low nibble = 1
    codes = np.full(256, 8, np.int64)
    for e, q in elems.items():
        codes[e] = q
    for g in range(8):
        c = codes[32 * g:32 * g + 32]
        b[8 + 16 * g:8 + 16 * g + 16] = (c[:16] | (c[16:] << 4)).astype(np.uint8)
    return b


# q4_0: lane l is the products 4l .. 4l + 3 of a block (code 9 is weight +1).
# q5_K: q4_K's lanes (element 4l of sub-block 0, scale 1).
# iq4_xs: lane l takes elements 4l .. 4l + 3 of every group (code 9 is level
# 13, the q8 value 1 gives 13 * (ls - 32) = 13; the expected 1 becomes 13).

def _dot_q4_0(blocks):
    xs, ys = [], []
    for s, ls in blocks:
        dx, dy = (4096.0, 8192.0) if s == BIG else (1.0, 1.0)
        xs.append(_q4_0(dx, {4 * l: 9 for l in ls}))
        ys.append(_q8_0(dy, {4 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_Q4_0, O.IMPL_AVX2, 32 * len(blocks), np.concatenate(xs), np.concatenate(ys))


def _dot_q5_K(blocks):
    xs, ys = [], []
    for s, ls in blocks:
        xs.append(_q5_K({4 * l: 1 for l in ls}, sc=[1]))
        ys.append(_q8_K(s, {4 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_Q5_K, O.IMPL_AVX2, 256 * len(blocks), np.concatenate(xs), np.concatenate(ys))


def _dot_iq4_xs(blocks):
    """Code 8 is level 1: the lane value is level * q8 = 1 * +-1."""
    xs, ys = [], []
    for s, ls in blocks:
        xs.append(_iq4_xs({}))
        ys.append(_q8_K(s, {4 * l: v for l, v in ls.items()}))
    return O.vec_dot(O.TYPE_IQ4_XS, O.IMPL_AVX2, 256 * len(blocks), np.concatenate(xs), np.concatenate(ys))


DOTS = [_dot_q4_K, _dot_q6_K, _dot_q8_0, _dot_q4_0, _dot_q5_K, _dot_iq4_xs]
DOT_IDS = ["q4_K", "q6_K", "q8_0", "q4_0", "q5_K", "iq4_xs"]


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("dot", DOTS, ids=DOT_IDS)
def test_avx2_dot_accumulation_order(dot, case):
    blocks, _ = CASES[case]
    assert dot(blocks) == 1.0


def test_avx2_dot_constructed_blocks_are_what_they_say():
    """The builders put the intended values where the golden-pinned generic
    dot and dequantizers see them: unit-scale blocks reproduce the integer
    sums (so a builder slip cannot make the order cases vacuous)."""
    for ls in ({0: 1}, {3: -1}, {7: 1, 2: 1}):
        x4 = _q4_K({4 * l: 1 for l in ls}, sc=[1])
        w = O.dequantize(O.TYPE_Q4_K, x4, 256)
        assert sorted(np.nonzero(w)[0].tolist()) == sorted(4 * l for l in ls) and np.all(w[w != 0] == 1.0)
        x6 = _q6_K({36 * l: 33 for l in ls}, sc=[1] * 16)
        w6 = O.dequantize(O.TYPE_Q6_K, x6, 256)
        nz = {e: w6[e] for e in np.nonzero(w6 + 32.0)[0]}  # every other code is 0 -> -32
        assert sorted(nz) == sorted(36 * l for l in ls) and all(v == 1.0 for v in nz.values())
        y = _q8_K(1.0, {36 * l: v for l, v in ls.items()})
        for t, x in ((O.TYPE_Q6_K, x6),):
            assert O.vec_dot(t, O.IMPL_GENERIC, 256, x, y) == float(sum(ls.values()))
        y4 = _q8_K(1.0, {4 * l: v for l, v in ls.items()})
        assert O.vec_dot(O.TYPE_Q4_K, O.IMPL_GENERIC, 256, x4, y4) == float(sum(ls.values()))
        x5 = _q5_K({4 * l: 1 for l in ls}, sc=[1])
        w5 = O.dequantize(O.TYPE_Q5_K, x5, 256)
        assert sorted(np.nonzero(w5)[0].tolist()) == sorted(4 * l for l in ls) and np.all(w5[w5 != 0] == 1.0)
        assert O.vec_dot(O.TYPE_Q5_K, O.IMPL_GENERIC, 256, x5, y4) == float(sum(ls.values()))
        x0 = _q4_0(1.0, {4 * l: 9 for l in ls})
        w0 = O.dequantize(O.TYPE_Q4_0, x0, 32)
        assert sorted(np.nonzero(w0)[0].tolist()) == sorted(4 * l for l in ls) and np.all(w0[w0 != 0] == 1.0)
        xi = _iq4_xs({})
        wi = O.dequantize(O.TYPE_IQ4_XS, xi, 256)
        assert np.all(wi[:32] == 1.0)  # level 1 times (ls - 32) = 1 in group 0
        assert O.vec_dot(O.TYPE_IQ4_XS, O.IMPL_GENERIC, 256, xi, y4) == float(sum(ls.values()))


def test_q4_K_avx2_min_lanes_fold_once_at_the_end():
    """q4_K keeps its mins in four lanes and adds them after hsum_float_8:
    block 0 puts 2^25 in lane 0 and -2^25 in min lane 0 (dmin = -y.d * 1, one
    min of 1 against a q8 block sum of 1), block 1 puts 1 in lane 1.  Then
    hsum = 2^25 + 1 -> 2^25 and the total is 0; folding the mins into the
    lanes (or per block) would give 1."""
    x0 = _q4_K({0: 1}, dmin=1.0, sc=[1], mins=[1])
    y0 = _q8_K(float(BIG), {0: 1})
    x1 = _q4_K({4: 1}, sc=[1])
    y1 = _q8_K(1.0, {4: 1})
    got = O.vec_dot(O.TYPE_Q4_K, O.IMPL_AVX2, 512, np.concatenate([x0, x1]), np.concatenate([y0, y1]))
    assert got == 0.0
    f = np.float32
    assert f(f(f(BIG) - f(BIG)) + f(1.0)) == 1.0  # the lanes-first alternative


def _fused_residual(d1, s1):
    """The exact product P = d1 * s1 (Fraction), its f32 rounding R, and the
    f32 value of P - R (exact: a fused multiply-add of d1, s1 onto an
    accumulator holding -R returns it; a separate multiply then add returns 0)."""
    from fractions import Fraction
    P = Fraction(float(d1)) * s1
    R = np.float32(float(P))  # P has at most 48 significant bits: exact in f64, one rounding to f32
    res = P - Fraction(float(R))
    assert res != 0 and np.float32(float(res)) == float(res)
    return R, np.float32(float(res))


@pytest.mark.parametrize("tname", ["q4_K", "q6_K"])
def test_avx2_kquant_dot_fuses_the_block_scale(tname):
    """acc = fma(d, float(sumi), acc): block 0 puts -R in lane 0 (d = -R,
    sumi 1), block 1 adds d1 * 3 with d1 = 1 + 2^-23, whose exact product P
    rounds to R.  Fused, lane 0 ends at P - R (a quarter ulp of 3, nonzero);
    a multiply then add would end at 0."""
    d1 = np.float32(1.0 + 2.0 ** -23)
    R, want = _fused_residual(d1, 3)
    if tname == "q4_K":
        xs = [_q4_K({0: 1}, sc=[1]), _q4_K({0: 1}, sc=[1])]
        ys = [_q8_K(-float(R), {0: 1}), _q8_K(float(d1), {0: 3})]
        t = O.TYPE_Q4_K
    else:
        xs = [_q6_K({0: 33}, sc=[1] * 16), _q6_K({0: 33}, sc=[1] * 16)]
        ys = [_q8_K(-float(R), {0: 1}), _q8_K(float(d1), {0: 3})]
        t = O.TYPE_Q6_K
    got = np.float32(O.vec_dot(t, O.IMPL_AVX2, 512, np.concatenate(xs), np.concatenate(ys)))
    assert got == want and want != 0


def test_avx2_q8_0_dot_fuses_the_block_scale():
    """q8_0's d = f16(x.d) * f16(y.d).  The last block has d1 = (1 + 2^-10)^2
    and lane 0 sum 255, an exact product P of 28 significant bits that rounds
    to R = m * 2^-16; the blocks before it put -R in lane 0 exactly, as
    d = 2^-8 * 2^-8 times lane sums 127 t + e adding up to -m (every partial
    sum a multiple of 2^-16 below 2^8, so exact).  Fused, the result is P - R;
    a multiply then add gives 0."""
    d1 = np.float32(np.float16(1.0 + 2.0 ** -10)) * np.float32(np.float16(1.0 + 2.0 ** -10))
    R, want = _fused_residual(d1, 255)
    m = int(round(float(R) * 2.0 ** 16))
    assert m * 2.0 ** -16 == float(R)
    xs, ys = [], []
    left = -m
    while left != 0:
        s = max(-48000, min(48000, left))
        t, e = divmod(s, 127) if s >= 0 else (-((-s) // 127), -((-s) % 127))
        assert 127 * t + e == s and abs(e) <= 127 and abs(t) <= 381
        # t over three codes of at most 127 against x codes of 127, e against a 1
        rest, parts = t, []
        for _ in range(3):
            p = max(-127, min(127, rest))
            parts.append(p)
            rest -= p
        assert rest == 0
        xs.append(_q8_0(2.0 ** -8, {0: 127, 1: 127, 2: 127, 3: 1}))
        ys.append(_q8_0(2.0 ** -8, {0: parts[0], 1: parts[1], 2: parts[2], 3: e}))
        left -= s
    xs.append(_q8_0(1.0 + 2.0 ** -10, {0: 127, 1: 127, 2: 1}))
    ys.append(_q8_0(1.0 + 2.0 ** -10, {0: 1, 1: 1, 2: 1}))
    n = 32 * len(xs)
    got = np.float32(O.vec_dot(O.TYPE_Q8_0, O.IMPL_AVX2, n, np.concatenate(xs), np.concatenate(ys)))
    assert got == want and want != 0


def test_q5_K_avx2_mins_fold_to_a_scalar_after_the_lanes():
    """q5_K folds each super-block's mins to a scalar, summs = fma(dmin,
    hsum, summs), added after hsum_float_8: block 0 puts 2^25 in lane 0 and
    -2^25 in summs, block 1 puts 1 in lane 1.  hsum = 2^25 + 1 -> 2^25, total
    0; mins folded into the lanes would give 1."""
    x0 = _q5_K({0: 1}, dmin=1.0, sc=[1], mins=[1])
    y0 = _q8_K(float(BIG), {0: 1})
    x1 = _q5_K({4: 1}, sc=[1])
    y1 = _q8_K(1.0, {4: 1})
    got = O.vec_dot(O.TYPE_Q5_K, O.IMPL_AVX2, 512, np.concatenate([x0, x1]), np.concatenate([y0, y1]))
    assert got == 0.0


@pytest.mark.parametrize("t", [O.TYPE_Q4_0, O.TYPE_Q5_K, O.TYPE_IQ4_XS, O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_Q8_0])
def test_avx2_dot_agrees_with_generic_on_normal_data(t):
    """Beside the order pins, the AVX2 arms give the golden-pinned generic
    dots' values up to float summation order, and their integer parts
    exactly (checked through unit scales by the pins above)."""
    rng = np.random.default_rng(int(t))
    nrows, K, ncols = 16, 1024, 3
    w = O.quantize_rows(t, (rng.standard_normal((nrows, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((ncols, K)).astype(np.float32)
    g = O.mul_mat(t, w, nrows, K, x, nth=2, impl=O.IMPL_GENERIC).astype(np.float64)
    a = O.mul_mat(t, w, nrows, K, x, nth=2, impl=O.IMPL_AVX2).astype(np.float64)
    tol = 1e-5 if t not in (O.TYPE_Q8_0, O.TYPE_Q4_0) else 1e-2  # q8_0 activations: AVX2 ties-to-even row quantizer
    assert np.max(np.abs(a - g)) <= tol * np.max(np.abs(g))
