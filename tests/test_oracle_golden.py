"""Pin the CPU oracle against the reference's own golden vectors.

Every value compared here was captured by the reference from its C build and
is committed in tests/golden/reference_goldens.json (extracted from
src/ggml/quants/golden.zig and src/ggml/cpu/quants/golden.zig).  A mismatch
means the restatement is wrong, not the golden.
"""
import json
import pathlib

import numpy as np
import pytest

import oracle_lib as O
from golden_patterns import QUANT_PATTERNS, VECDOT_PATTERNS, quant_imatrix, quant_src, vecdot_fill

G = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_goldens.json").read_text())
QREC = {(r["name"], r["pattern"]): r for r in G["quant"]["records"]}
N_PER_ROW, N_ROWS = G["quant"]["n_per_row"], G["quant"]["n_rows"]
N_ELEM = N_PER_ROW * N_ROWS


@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q8_1", "Q8_K", "IQ4_XS"])
@pytest.mark.parametrize("pattern", QUANT_PATTERNS)
def test_quantize_ref_matches_golden(name, pattern):
    """quants/k.zig:774-829 and legacy.zig:682-751 checkK/checkLegacy."""
    rec = QREC[(name, pattern)]
    t = O.TYPE_IDS[name]
    src = quant_src(pattern, N_ROWS, N_PER_ROW)
    q = O.quantize_ref(t, src)
    assert q.nbytes == rec["row_size"] * N_ROWS
    assert O.fnv1a(q) == rec["ref"], f"{name}/{pattern} quantize bytes differ"
    if "deq" in rec:
        deq = O.dequantize(t, q, N_ELEM)
        assert O.fnv1a(deq) == rec["deq"], f"{name}/{pattern} dequantize floats differ"


@pytest.mark.parametrize("name", ["Q4_0", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS"])
@pytest.mark.parametrize("pattern", QUANT_PATTERNS)
def test_quantize_chunk_matches_golden(name, pattern):
    """quants/chunks.zig:758-790 checkChunk, with and without an importance matrix."""
    rec = QREC[(name, pattern)]
    t = O.TYPE_IDS[name]
    src = quant_src(pattern, N_ROWS, N_PER_ROW)
    out = O.quantize_chunk(t, src, N_ROWS, N_PER_ROW)
    assert out.nbytes == rec["chunk_bytes"]
    assert O.fnv1a(out) == rec["chunk"]
    out = O.quantize_chunk(t, src, N_ROWS, N_PER_ROW, quant_imatrix(N_PER_ROW))
    assert O.fnv1a(out) == rec["chunk_imatrix"], f"{name}/{pattern} imatrix chunk differs"


@pytest.mark.parametrize("row", ["q8_0", "q8_1", "q8_K"])
@pytest.mark.parametrize("pattern", VECDOT_PATTERNS)
def test_row_quantizers_match_golden(row, pattern):
    """cpu/quants/testing.zig checkRow: FNV of the bytes over 512 elements."""
    want = G["vecdot"]["rows"]["row_" + row][pattern]
    x, _ = vecdot_fill(pattern)
    t = O.TYPE_IDS[row.upper().replace("Q8_K", "Q8_K")] if row != "q8_K" else O.TYPE_Q8_K
    q = O.quantize_ref(t, x)
    assert O.fnv1a(q) == want


@pytest.mark.parametrize("kern", ["q8_0", "q4_0", "q4_K", "q5_K", "q6_K", "iq4_xs"])
@pytest.mark.parametrize("pattern", VECDOT_PATTERNS)
def test_vec_dot_generic_matches_golden(kern, pattern):
    """cpu/quants/testing.zig check: x via ggml_quantize_chunk(imatrix = ones),
    y via the vec_dot_type's reference quantizer; raw f32 bits compared."""
    want = G["vecdot"]["dots"][kern][pattern]
    n = G["vecdot"]["nelem"]
    x, y = vecdot_fill(pattern, n)
    t = O.TYPE_IDS[kern.upper().replace("_K", "_K")]
    yt = O.TYPE_Q8_0 if t in (O.TYPE_Q8_0, O.TYPE_Q4_0) else O.TYPE_Q8_K
    xq = O.quantize_chunk(t, x, 1, n, np.ones(n, dtype=np.float32))
    yq = O.quantize_ref(yt, y)
    got = np.float32(O.vec_dot(t, O.IMPL_GENERIC, n, xq, yq)).view(np.uint32)
    assert int(got) == want, f"{kern}/{pattern}: got {got:#010x} want {want:#010x}"


def test_nearest_int_is_half_to_even():
    """quants/helpers.zig:651-669."""
    L = O.lib()
    for v, want in [(0.5, 0), (1.5, 2), (2.5, 2), (3.5, 4), (-0.5, 0), (-1.5, -2), (3.2, 3), (3.7, 4), (-3.2, -3)]:
        assert L.orc_nearest_int(v) == want


def test_fp16_roundtrip_all_halves():
    """fp16 -> fp32 -> fp16 is the identity on every non-NaN half, and the
    narrowing agrees with numpy's IEEE round-to-nearest-even."""
    L = O.lib()
    for h in range(0, 0x10000, 7):
        f = L.orc_fp16_to_fp32(h)
        if np.isnan(f):
            continue
        assert L.orc_fp16_to_fp32(h) == np.uint16(h).view(np.float16).astype(np.float32)
        assert L.orc_fp32_to_fp16(f) == h
    rng = np.random.default_rng(0)
    for v in rng.standard_normal(2000).astype(np.float32) * np.float32(3e3):
        assert L.orc_fp32_to_fp16(float(v)) == int(np.float16(v).view(np.uint16))
