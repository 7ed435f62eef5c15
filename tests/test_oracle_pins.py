"""Pins for the oracle functions the reference's golden vectors do not cover
directly.  Each check ties a function to golden-pinned ones (the reference
quantizers, dequantizers and generic dot products, test_oracle_golden.py) or
to a closed form, so that a wrong index, a transposed operand or a dropped
term fails here:

- orc_block_dots_q8_1: on blocks whose super-block scale is 1 and whose
  minimum is 0, the golden-pinned dequantizer returns sc * q exactly, so each
  integer block dot is (sum of dequantized weight * q8) / sc;
- orc_mul_mat_q8_1_f64: with activations whose Q8_1 block sums are zero it is
  the f64 dot of the dequantized weights and dequantized activations; with
  d = 0 weights only the min term remains, equal up to the f16 rounding of s;
- orc_mul_mat (generic): each output is the golden-pinned vec_dot of the
  weight row with the activation column quantized by the golden-pinned
  quantize_row_q8_K_ref / q8_0_ref, and no output depends on the thread count;
- orc_mul_mat_id: every (token, slot) row is orc_mul_mat of the routed expert
  and the routed activation row; ids of -1 give zero rows;
- the AVX2 restatements (no x86 goldens exist in the reference): checked
  against the generic ones, integers exact and floats within rounding;
- orc_fill_normal: moments of the distribution and a committed fingerprint of
  the seeded stream (determinism across machines);
- orc_tinyblas_q0 (x86 Q8_0 / Q4_0 GEMM): with unit scales every output is the
  exact integer dot (numpy), which pins the lane grouping, the Q4_0 nibble
  order and offset and the block / column indexing; one case whose lanes hold
  2^24, -2^24 and 1 sums to exactly 1 only in the reference's horizontal order
  ((h0 + h2) + (h1 + h3), h = upper + lower half), where a sequential or
  adjacent-pair order loses the 1; on quantized normal data it agrees with the
  golden-pinned vec_dot route within rounding and does not depend on threads.
"""
import numpy as np
import pytest

import oracle_lib as O

RNG = np.random.default_rng(1234)
F16_ONE = np.float16(1.0).view(np.uint16)


def _q8_1(x):
    """AoS Q8_1 blocks of one row and the int8 values, per 32."""
    y = O.quantize_ref(O.TYPE_Q8_1, x).reshape(-1, 36)
    q = y[:, 4:].view(np.int8).astype(np.int64)
    d = y[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    return y.reshape(-1), q, d


def _unit_q4_k_blocks(nblocks):
    """Q4_K blocks with d = 1, dmin = 0, random 6-bit scales and random
    nibbles: dequantized weight = sc_j * q."""
    b = RNG.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    b[:, 2:4] = 0
    return b


def _unit_q5_k_blocks(nblocks):
    """Q5_K likewise: dequantized weight = sc_j * (q + 16 h)."""
    b = RNG.integers(0, 256, size=(nblocks, 176), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    b[:, 2:4] = 0
    return b


def _unit_q6_k_blocks(nblocks):
    b = RNG.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    b[:, 208:210] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    return b


def _unit_q4_0_blocks(nblocks):
    """Q4_0 with d = 1: dequantized weight = q - 8, the block dot's operand."""
    b = RNG.integers(0, 256, size=(nblocks, 18), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    return b


def _unit_iq4_xs_blocks(nblocks):
    """IQ4_XS with d = 1, random 6-bit scales and random level indices:
    dequantized weight = (ls - 32) * level[q]."""
    b = RNG.integers(0, 256, size=(nblocks, 136), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    return b


def _unit_q8_0_blocks(nblocks):
    b = RNG.integers(0, 256, size=(nblocks, 34), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(F16_ONE.tobytes(), dtype=np.uint8)
    return b


@pytest.mark.parametrize("t,maker,group", [(O.TYPE_Q4_K, _unit_q4_k_blocks, 32),
                                           (O.TYPE_Q5_K, _unit_q5_k_blocks, 32),
                                           (O.TYPE_Q6_K, _unit_q6_k_blocks, 16),
                                           (O.TYPE_Q8_0, _unit_q8_0_blocks, 32),
                                           (O.TYPE_Q4_0, _unit_q4_0_blocks, 32),
                                           (O.TYPE_IQ4_XS, _unit_iq4_xs_blocks, 32)])
def test_block_dots_against_unit_scale_dequantization(t, maker, group):
    nrows, K = 3, 512
    bs = 32 if t in (O.TYPE_Q8_0, O.TYPE_Q4_0) else 256
    w = maker(nrows * K // bs).reshape(nrows, -1)
    x = RNG.standard_normal(K).astype(np.float32) * 3
    y, q8, _ = _q8_1(x)
    got = O.block_dots_q8_1(t, w, nrows, K, np.tile(y, 1))
    q8 = q8.reshape(-1)
    checked = 0
    for r in range(nrows):
        deq = O.dequantize(t, w[r], K).astype(np.float64)  # = scale * q, exactly
        for j in range(K // group):
            sl = slice(group * j, group * (j + 1))
            # the sub-block's integer scale: deq / q for any nonzero code; the
            # scale itself comes from the golden-pinned dequantizer
            prod = float(np.dot(deq[sl], q8[sl]))
            if t in (O.TYPE_Q8_0, O.TYPE_Q4_0):
                assert got[r, j] == prod
                checked += 1
                continue
            sc = _scale_of(t, w[r], j)
            if sc == 0:
                continue
            assert prod == sc * got[r, j], (r, j)
            checked += 1
    assert checked > nrows * (K // group) // 2


def _scale_of(t, row, j):
    """Sub-block scale of a unit-scale block, read back through the
    dequantizer: a block whose codes are all 1 (Q4_K, Q5_K), all 33 (Q6_K) or
    all index 8 (IQ4_XS, level 1) dequantizes to the scale itself."""
    bs = {O.TYPE_Q4_K: 144, O.TYPE_Q5_K: 176, O.TYPE_Q6_K: 210, O.TYPE_IQ4_XS: 136}[t]
    blk = row.reshape(-1, bs)[j // (16 if t == O.TYPE_Q6_K else 8)].copy()
    if t == O.TYPE_IQ4_XS:
        blk[8:] = 0x88  # every index 8, level 1
        deq = O.dequantize(t, blk, 256)
        return deq[32 * (j % 8)]
    if t == O.TYPE_Q4_K:
        blk[16:] = 0x11  # every nibble 1
        deq = O.dequantize(t, blk, 256)
        return deq[32 * (j % 8)]
    if t == O.TYPE_Q5_K:
        blk[16:48] = 0  # no fifth bits
        blk[48:] = 0x11  # every nibble 1
        deq = O.dequantize(t, blk, 256)
        return deq[32 * (j % 8)]
    blk[0:128] = 0x11  # low 4 bits 1
    blk[128:192] = 0xAA  # high 2 bits 2 -> code 33, value sc * 1
    deq = O.dequantize(t, blk, 256)
    sub = j % 16
    return deq[16 * sub]


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_Q8_0, O.TYPE_Q4_0, O.TYPE_IQ4_XS])
def test_mul_mat_q8_1_f64_is_the_dequantized_dot(t):
    nrows, K, ncols = 5, 768, 3
    w = O.quantize_rows(t, RNG.standard_normal((nrows, K)).astype(np.float32) * 0.02)
    # pairwise-negated activations: every Q8_1 block sum is 0, so s = 0 exactly
    half = RNG.standard_normal((ncols, K // 2)).astype(np.float32)
    x = np.empty((ncols, K), dtype=np.float32)
    x[:, 0::2], x[:, 1::2] = half, -half
    ys, deq_y = [], []
    for c in range(ncols):
        y, q8, d = _q8_1(x[c])
        assert np.all(q8.sum(axis=1) == 0)
        ys.append(y)
        deq_y.append((q8 * d[:, None]).reshape(-1))
    got = O.mul_mat_q8_1_f64(t, w, nrows, K, np.stack(ys), ncols)
    deq_w = np.stack([O.dequantize(t, w[r], K).astype(np.float64) for r in range(nrows)])
    want = np.stack(deq_y) @ deq_w.T
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())


@pytest.mark.parametrize("t,bs", [(O.TYPE_Q4_K, 144), (O.TYPE_Q5_K, 176)])
def test_mul_mat_q8_1_f64_min_term(t, bs):
    """d = 0: a Q4_K / Q5_K weight is -dmin*m_j on its sub-block, and the
    formula's min term uses s = f16(d8 * sum q) in place of d8 * sum q."""
    nrows, K = 4, 512
    w = O.quantize_rows(t, RNG.standard_normal((nrows, K)).astype(np.float32) * 0.02)
    w = w.reshape(nrows, -1, bs).copy()
    w[:, :, 0:2] = 0  # d = 0
    w = w.reshape(nrows, -1)
    x = RNG.standard_normal(K).astype(np.float32) + 0.3
    y, q8, d = _q8_1(x)
    got = O.mul_mat_q8_1_f64(t, w, nrows, K, y[None, :], 1)[0]
    deq_y = (q8 * d[:, None]).reshape(-1)
    for r in range(nrows):
        deq = O.dequantize(t, w[r], K).astype(np.float64)
        per_block = (deq * deq_y).reshape(-1, 32).sum(axis=1)
        want = per_block.sum()
        bound = 2.0 ** -11 * np.abs(per_block).sum() + 1e-30
        assert abs(got[r] - want) <= bound, (r, got[r], want, bound)
        assert abs(want) > 10 * bound  # the min term is really there


VDT = {O.TYPE_Q4_K: O.TYPE_Q8_K, O.TYPE_Q5_K: O.TYPE_Q8_K, O.TYPE_Q6_K: O.TYPE_Q8_K, O.TYPE_Q8_0: O.TYPE_Q8_0,
       O.TYPE_Q4_0: O.TYPE_Q8_0, O.TYPE_IQ4_XS: O.TYPE_Q8_K}


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_Q8_0, O.TYPE_Q4_0, O.TYPE_IQ4_XS])
def test_mul_mat_generic_is_vec_dot_per_output(t):
    nrows, K, ncols = 7, 512, 4
    w = O.quantize_rows(t, RNG.standard_normal((nrows, K)).astype(np.float32) * 0.02)
    x = RNG.standard_normal((ncols, K)).astype(np.float32)
    got = O.mul_mat(t, w, nrows, K, x, nth=3)
    for c in range(ncols):
        yq = O.quantize_ref(VDT[t], x[c])
        for r in range(nrows):
            assert got[c, r] == np.float32(O.vec_dot(t, O.IMPL_GENERIC, K, w[r], yq)), (c, r)
    for nth in (1, 2, 8):
        assert np.array_equal(O.mul_mat(t, w, nrows, K, x, nth=nth), got)


@pytest.mark.parametrize("ne11", [1, 2])
def test_mul_mat_id_is_mul_mat_per_slot(ne11):
    t, n_as, nrows, K, n_tokens, n_ids = O.TYPE_Q4_K, 5, 6, 256, 4, 2
    w = O.quantize_rows(t, RNG.standard_normal((n_as * nrows, K)).astype(np.float32) * 0.02).reshape(n_as, nrows, -1)
    x = RNG.standard_normal((n_tokens, ne11, K)).astype(np.float32)
    ids = RNG.integers(-1, n_as, size=(n_tokens, n_ids)).astype(np.int32)
    ids[0, 0] = -1
    got = O.mul_mat_id(t, w, n_as, nrows, K, x, ids, nth=3)
    for tok in range(n_tokens):
        for s in range(n_ids):
            e = ids[tok, s]
            if e < 0:
                assert np.all(got[tok, s] == 0)
                continue
            want = O.mul_mat(t, w[e], nrows, K, x[tok, s % ne11][None, :], nth=1)[0]
            assert np.array_equal(got[tok, s], want), (tok, s)


@pytest.mark.skipif(not O.has_avx2(), reason="host has no AVX2")
@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_Q8_0])
def test_avx2_restatement_agrees_with_generic(t):
    """Parity unpinned against the reference (no x86 goldens): the AVX2 path
    is held to the golden-pinned generic one, up to float summation order."""
    nrows, K, ncols = 16, 1024, 3
    w = O.quantize_rows(t, RNG.standard_normal((nrows, K)).astype(np.float32) * 0.02)
    x = RNG.standard_normal((ncols, K)).astype(np.float32)
    g = O.mul_mat(t, w, nrows, K, x, nth=2, impl=O.IMPL_GENERIC).astype(np.float64)
    a = O.mul_mat(t, w, nrows, K, x, nth=2, impl=O.IMPL_AVX2).astype(np.float64)
    assert np.max(np.abs(a - g)) <= 1e-5 * np.max(np.abs(g))


def test_q8_0_avx2_row_quantizer_against_ref():
    x = RNG.standard_normal(4096).astype(np.float32)
    ref = O.quantize_ref(O.TYPE_Q8_0, x).reshape(-1, 34)
    avx = np.zeros_like(ref)
    lib = O.lib()
    lib.orc_quantize_row_q8_0_avx2(x.ctypes.data, avx.ctypes.data, x.size)
    assert np.array_equal(ref[:, 0:2], avx[:, 0:2])  # same scale d = amax / 127
    dq = ref[:, 2:].view(np.int8).astype(int) - avx[:, 2:].view(np.int8).astype(int)
    assert np.abs(dq).max() <= 1 and np.count_nonzero(dq) <= x.size // 100  # rounding ties only


def test_fill_normal_moments_and_fingerprint():
    v = O.fill_normal(42, 1 << 20).astype(np.float64)
    assert abs(v.mean()) < 5 / np.sqrt(v.size)
    assert abs(v.std() - 1.0) < 5 / np.sqrt(2 * v.size)
    assert abs((v ** 3).mean()) < 0.02 and abs((v ** 4).mean() - 3.0) < 0.05
    assert O.fill_normal(42, 8, 0.0, 0.02)[0] == np.float32(O.fill_normal(42, 8)[0] * np.float32(0.02))
    # fingerprints of the seeded streams the configs use (weights 42, activations 43, router 44)
    fp = {s: O.fnv1a(O.fill_normal(s, 4096)) for s in (42, 43, 44)}
    assert fp == FINGERPRINTS


FINGERPRINTS = {42: 3664293373807877317, 43: 7632513219039429954, 44: 984130064333561219}


@pytest.mark.parametrize("n", [1, 2, 7, 4096, (1 << 20) + 3])
def test_threaded_generators_equal_serial(n):
    """The threaded normal fill (split at even indices, each part seeded from
    its first pair's SplitMix64 state) and the threaded row quantizer give the
    serial generators' values exactly, for odd lengths and ragged splits."""
    serial = O.fill_normal(42, n, 0.0, 0.02, nth=1)
    for nth in (2, 3, 8):
        assert np.array_equal(O.fill_normal(42, n, 0.0, 0.02, nth=nth), serial)
    rows = RNG.standard_normal((13, 512)).astype(np.float32) * 0.02
    for t in (O.TYPE_Q4_K, O.TYPE_Q6_K, O.TYPE_Q8_0):
        one = O.quantize_ref(t, rows.reshape(-1)).reshape(13, -1)
        for nth in (1, 4, 16):
            assert np.array_equal(O.quantize_rows(t, rows, nth=nth), one)


TILED = [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_IQ4_XS]


def _random_blocks(t, nrows, K, rng):
    """Random bytes as blocks with a modest finite fp16 scale, as the
    reference's tiled test builds them (tiled.zig:1323-1343)."""
    bs, bb = O.BLOCK[t]
    nb = nrows * K // bs
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    scale = (0x3000 | (rng.integers(0, 1 << 16, size=nb) & 0x03FF)).astype(np.uint16)
    if t == O.TYPE_Q6_K:
        blk[:, bb - 2:bb] = scale.view(np.uint8).reshape(nb, 2)
    else:
        blk[:, 0:2] = scale.view(np.uint8).reshape(nb, 2)
        if t in (O.TYPE_Q4_K, O.TYPE_Q5_K):
            blk[:, 2:4] = (scale ^ 0x0100).view(np.uint8).reshape(nb, 2)
    return blk.reshape(nrows, -1)


@pytest.mark.skipif(not O.has_avx2(), reason="the tiled path is the AVX2 arm")
@pytest.mark.parametrize("t", TILED)
@pytest.mark.parametrize("K,nrows,ncols", [(512, 40, 33), (768, 24, 5)])
def test_tiled_gemm_agrees_with_vec_dot(t, K, nrows, ncols):
    """The reference's own check (checkMulMat, tiled.zig:1367-1438): every
    element within 2e-4 x max|out| of vec_dot on the same Q8_K rows, on the
    standard path (33 columns: a ragged 16-row and 16-column tail) and the
    narrow one (5 columns, K in two- and one-slab extents), for random blocks
    and for quantized N(0, 0.02) weights."""
    rng = np.random.default_rng(0x711ED + t + K)
    x = (rng.random((ncols, K), dtype=np.float32) * 2 - 1).astype(np.float32)
    for wq in (_random_blocks(t, nrows, K, rng),
               O.quantize_rows(t, rng.standard_normal((nrows, K)).astype(np.float32) * 0.02)):
        got = O.mul_mat_tiled(t, wq, nrows, K, x, nth=1)
        want = np.zeros_like(got)
        for j in range(ncols):
            y = O.quantize_ref(O.TYPE_Q8_K, x[j])
            for i in range(nrows):
                want[j, i] = O.vec_dot(t, O.IMPL_GENERIC, K, wq[i], y)
        scale = float(np.max(np.abs(got)))
        assert scale > 0 and np.all(np.isfinite(got))
        assert np.max(np.abs(got - want)) <= 2e-4 * scale


@pytest.mark.skipif(not O.has_avx2(), reason="the tiled path is the AVX2 arm")
@pytest.mark.parametrize("t", TILED)
def test_tiled_gemm_is_independent_of_threads_and_windows(t):
    """Each output adds its slabs' terms in K order whatever the chunking, the
    window or the path: the same bits on 1, 3 and 8 threads (other chunk
    sizes, 256-row windows on 300 rows), and a column alone (the narrow
    path) equals that column inside a wide run (the standard path)."""
    rng = np.random.default_rng(77 + t)
    nrows, K, ncols = 300, 1024, 40
    wq = O.quantize_rows(t, rng.standard_normal((nrows, K)).astype(np.float32) * 0.02)
    x = rng.standard_normal((ncols, K)).astype(np.float32)
    one = O.mul_mat_tiled(t, wq, nrows, K, x, nth=1)
    for nth in (3, 8):
        assert np.array_equal(O.mul_mat_tiled(t, wq, nrows, K, x, nth=nth), one)
    narrow = O.mul_mat_tiled(t, wq, nrows, K, x[17:20], nth=2)
    assert np.array_equal(narrow, one[17:20])
    # and the whole result is the CPU mul_mat's within the NMSE gate
    cpu = O.mul_mat(t, wq, nrows, K, x, nth=4)
    assert float(np.sum((one.astype(np.float64) - cpu) ** 2) / np.sum(cpu.astype(np.float64) ** 2)) < 1e-10


def test_tiled_gemm_declines_untiled_types():
    wq = O.quantize_rows(O.TYPE_Q8_0, np.zeros((16, 256), np.float32))
    assert O.mul_mat_tiled(O.TYPE_Q8_0, wq, 16, 256, np.zeros((8, 256), np.float32)) is None


# ---------------------------------------------------------------- tinyBLAS (x86 Q8_0 / Q4_0 GEMM)

Q80 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
Q40 = np.dtype([("d", "<u2"), ("qs", "u1", 16)])


def _q8_0_blocks(vals, d=F16_ONE):
    """int8 values [rows, K] -> Q8_0 blocks with scale d."""
    rows, K = vals.shape
    b = np.zeros((rows, K // 32), dtype=Q80)
    b["d"] = d
    b["qs"] = vals.reshape(rows, K // 32, 32)
    return b


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_0])
def test_tinyblas_exact_on_unit_scales(t):
    rng = np.random.default_rng(77 + t)
    nrows, K, ncols = 13, 256, 5
    if t == O.TYPE_Q8_0:
        wv = rng.integers(-127, 128, size=(nrows, K)).astype(np.int8)
        w = _q8_0_blocks(wv)
    else:
        wv = rng.integers(-8, 8, size=(nrows, K)).astype(np.int8)
        nib = (wv + 8).astype(np.uint8).reshape(nrows, K // 32, 32)
        w = np.zeros((nrows, K // 32), dtype=Q40)
        w["d"] = F16_ONE
        w["qs"] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    yv = rng.integers(-127, 128, size=(ncols, K)).astype(np.int8)
    y = _q8_0_blocks(yv)
    got = O.tinyblas_q0(t, w.view(np.uint8), nrows, K, y.view(np.uint8), ncols, nth=3)
    want = (yv.astype(np.int64) @ wv.astype(np.int64).T).astype(np.float64)
    np.testing.assert_array_equal(got.astype(np.float64), want)


def test_tinyblas_horizontal_sum_order():
    K = 64
    w = np.zeros((1, 2), dtype=Q80)
    y = np.zeros((1, 2), dtype=Q80)
    big = np.float16(2048.0).view(np.uint16)  # 2048 * 2048 = 2^22
    w[0, 0]["d"], y[0, 0]["d"] = big, big
    w[0, 0]["qs"][0], y[0, 0]["qs"][0] = 4, 1     # lane 0: 4 * 2^22 = 2^24
    w[0, 0]["qs"][16], y[0, 0]["qs"][16] = -4, 1  # lane 4: -2^24
    w[0, 1]["d"], y[0, 1]["d"] = F16_ONE, F16_ONE
    w[0, 1]["qs"][4], y[0, 1]["qs"][4] = 1, 1     # lane 1: 1
    got = O.tinyblas_q0(O.TYPE_Q8_0, w.view(np.uint8), 1, K, y.view(np.uint8), 1)
    assert got[0, 0] == 1.0  # exact; ((L0 + L1) + ...) or ((L0 + L1) + (L2 + L3)) + ... give 0


@pytest.mark.skipif(not O.has_avx2(), reason="the tinyBLAS path is the x86 AVX2 arm")
@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_0])
def test_tinyblas_agrees_with_vec_dot_route(t):
    nrows, K, ncols = 48, 1024, 7
    wq = O.quantize_rows(t, O.fill_normal(31 + t, nrows * K, 0.0, 0.02).reshape(nrows, K))
    x = O.fill_normal(41 + t, ncols * K).reshape(ncols, K)
    tb = O.mul_mat_tinyblas(t, wq, nrows, K, x, nth=1)
    vd = O.mul_mat(t, wq, nrows, K, x, nth=2, impl=O.IMPL_AVX2)
    scale = np.abs(vd).max()
    assert np.abs(tb - vd).max() <= 2e-6 * scale
    np.testing.assert_array_equal(O.mul_mat_tinyblas(t, wq, nrows, K, x, nth=5), tb)
    assert O.mul_mat_tinyblas(t, wq, nrows, K, x[:1]) is None  # llamafile_sgemm declines one column
    assert O.mul_mat_tinyblas(O.TYPE_Q4_K, O.quantize_rows(O.TYPE_Q4_K, O.fill_normal(1, 256 * 8).reshape(8, 256)),
                              8, 256, x[:, :256]) is None


@pytest.mark.skipif(not O.has_avx2(), reason="host has no AVX2")
@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_0])
def test_tinyblas_tile_loops_equal_the_per_output_restatement(t):
    """The timing-faithful tile loops (mnpack over gemm4xN / gemmMx4 / gemm,
    each splitting its tiles over the threads, sgemm.zig:667-880) give every
    output the per-output restatement's value bit for bit, on shapes whose
    remainders reach every tile kernel (1-13 rows and columns past the 4 x 2
    tiles), at 1-7 threads, with every output written exactly once (NaN
    prefill)."""
    rng = np.random.default_rng(17)
    K = 96
    for nrows in (1, 2, 3, 4, 5, 6, 7, 9, 13, 33):
        for ncols in (1, 2, 3, 4, 5, 7, 13):
            w = O.quantize_rows(t, (rng.standard_normal((nrows, K)) * 0.02).astype(np.float32))
            y = O.quantize_rows(O.TYPE_Q8_0, rng.standard_normal((ncols, K)).astype(np.float32))
            want = O.tinyblas_q0_per_output(t, w, nrows, K, y, ncols, nth=1)
            for nth in (1, 3, 7):
                got = O.tinyblas_q0(t, w, nrows, K, y, ncols, nth=nth)
                assert np.all(np.isfinite(got)), (nrows, ncols, nth)
                np.testing.assert_array_equal(got, want, err_msg=f"{nrows}x{ncols} nth={nth}")
