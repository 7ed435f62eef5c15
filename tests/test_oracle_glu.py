"""CPU oracle of the GLU ops (orc_glu_f32), pinned against:
  - the reference's known answers (src/ggml/cpu/ops/vecinline.zig:733-760:
    x = {-2, -0.5, 0, 0.5, 2, 12, -12, 3}, g = {1..8}: reglu y[0] = 0,
    y[4] = 10; geglu y[5] = 72; gelu y[5] = 12, y[6] = 0);
  - closed forms evaluated independently in double precision (Python's math
    module and numpy's float16 rounding), which fix the formulas, the clamp
    sides, where alpha enters and which operand gates;
  - the NaN behaviour of std::min / std::clamp the reference tests
    (src/ggml/cpu/ops/activation.zig, "std::min and std::clamp pass a NaN
    through").
The oracle is test infrastructure: it checks the device GLU, it is never the
thing measured."""
import math

import numpy as np
import pytest

import oracle_lib as O

X = np.array([-2, -0.5, 0, 0.5, 2, 12, -12, 3], np.float32)
G = np.arange(1, 9, dtype=np.float32)


def ulps(a, b):
    """Distance in float32 ulps (of the larger magnitude)."""
    a, b = np.float32(a), np.float32(b)
    if a == b:
        return 0.0
    return abs(float(a) - float(b)) / float(np.spacing(np.float32(max(abs(a), abs(b)))))


def test_reference_known_answers():
    reglu = O.glu(O.GLU_REGLU, X, G)
    assert reglu[0] == 0 and reglu[4] == 10
    geglu = O.glu(O.GLU_GEGLU, X, G)
    assert geglu[5] == 72  # x >= 10: x * g
    gelu = O.glu(O.GLU_GEGLU, X, np.ones(8, np.float32))
    assert gelu[5] == 12 and gelu[6] == 0  # x >= 10 passes, x <= -10 is zero


def silu(x):
    return x / (1.0 + math.exp(-x))


def test_swiglu_closed_form():
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(4000) * 4).astype(np.float32)
    u = rng.standard_normal(4000).astype(np.float32)
    got = O.glu(O.GLU_SWIGLU, g, u)
    for gi, ui, yi in zip(g, u, got):
        assert ulps(yi, silu(float(gi)) * float(ui)) <= 3
    # the gate is the first operand: swapping changes the result
    assert not np.allclose(O.glu(O.GLU_SWIGLU, u, g), got)


def gelu_table(x):
    """f16(gelu(f16(x))) with the CPU's f32 operation order emulated in
    numpy float32 (the inner 1 + a*x*x as one rounding: exact in double, then
    rounded), tanh correctly rounded to f32, and numpy's float16 rounding."""
    f = np.float32
    t = f(np.float16(x))
    fma = f(float(f(f(0.044715) * t)) * float(t) + 1.0)
    inner = f(f(f(0.79788456080286535587989211986876) * t) * fma)
    th = f(math.tanh(float(inner)))
    return float(np.float16(f(f(f(0.5) * t) * f(f(1.0) + th))))


def test_geglu_table_path():
    # every f16 value in (-10, 10), once: the table the CPU builds
    h = np.arange(0, 1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h) & (h > -10) & (h < 10)]
    got = O.glu(O.GLU_GEGLU, h, np.ones_like(h))
    want = np.array([gelu_table(v) for v in h], np.float32)
    diff = got != want
    # libm's tanhf is not always correctly rounded; near x = -10 the f32 sum
    # 1 + tanh cancels, so its last ulp can move the f16 result by one step
    assert diff.mean() < 5e-3, diff.mean()
    sp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(got - want)[diff] <= sp[diff] * 1.0001)
    assert np.all(h[diff] < -2.0)  # only where the sum cancels
    # gelu itself (f32) against double precision where 1 + tanh does not cancel
    for v in (-0.7, 0.3, 1.9, 4.5):
        inner = 0.79788456080286535587989211986876 * v * (1.0 + 0.044715 * v * v)
        assert ulps(O.gelu_f32(v), 0.5 * v * (1.0 + math.tanh(inner))) <= 4
    # the gate, not the value, goes through gelu
    assert O.glu(O.GLU_GEGLU, np.float32([2.0]), np.float32([3.0]))[0] == np.float32(gelu_table(2.0) * 3.0)


def oai(g, u, alpha, limit):
    x = min(g, limit)
    y = max(-limit, min(u, limit))
    arg = float(np.float32(alpha) * np.float32(-x))  # the f32 product the CPU rounds
    return x / (1.0 + math.exp(arg)) * (y + 1.0)


def clamp_glu(g, u, limit):
    x = min(g, limit)
    y = max(-limit, min(u, limit))
    return x / (1.0 + math.exp(-x)) * y


@pytest.mark.parametrize("alpha,limit", [(1.702, 7.0), (0.5, 3.0)])
def test_swiglu_oai_and_clamp_closed_forms(alpha, limit):
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(3000) * 6).astype(np.float32)
    u = (rng.standard_normal(3000) * 6).astype(np.float32)
    got = O.glu(O.GLU_SWIGLU_OAI, g, u, alpha, limit)
    for gi, ui, yi in zip(g, u, got):
        assert ulps(yi, oai(float(gi), float(ui), float(np.float32(alpha)), float(np.float32(limit)))) <= 4
    got = O.glu(O.GLU_SWIGLU_CLAMP, g, u, 0.0, limit)
    for gi, ui, yi in zip(g, u, got):
        assert ulps(yi, clamp_glu(float(gi), float(ui), float(np.float32(limit)))) <= 4
    # the gate is capped from above only, the value on both sides
    big = O.glu(O.GLU_SWIGLU_CLAMP, np.float32([50.0, 50.0]), np.float32([50.0, -50.0]), 0.0, limit)
    want = np.float32(limit / (1.0 + math.exp(-limit)) * limit)
    assert ulps(big[0], want) <= 4 and ulps(big[1], -want) <= 4
    # alpha scales the sigmoid's argument: a different alpha changes the result
    assert O.glu(O.GLU_SWIGLU_OAI, np.float32([1.0]), np.float32([1.0]), 1.0, limit)[0] != \
        O.glu(O.GLU_SWIGLU_OAI, np.float32([1.0]), np.float32([1.0]), 2.0, limit)[0]


def test_nan_passes_through_min_and_clamp():
    nan = np.float32(np.nan)
    for op in (O.GLU_SWIGLU_OAI, O.GLU_SWIGLU_CLAMP):
        assert np.isnan(O.glu(op, np.float32([nan]), np.float32([1.0]), 1.702, 7.0)[0])
        assert np.isnan(O.glu(op, np.float32([1.0]), np.float32([nan]), 1.702, 7.0)[0])


# ---------------------------------------------------------------- SWIGLU's vector arm
#
# On an x86 AVX2 host ggml_vec_swiglu_f32 runs 8-lane steps of
# ggml_v_silu(x) * g, whose exp is ARM's optimised expf routine
# (src/ggml/cpu/vec.zig:537-599; upstream records its maximum error as
# 1.45358 + 0.5 ulp), and the scalar x / (1 + expf(-x)) * g for the last
# nc % 8 of each row.  The reference holds no golden for either.  The
# restatement (orc_v_expf) is pinned to the routine's published error bound
# over its whole range, to its exact points and to its range limits, so a
# dropped or misplaced polynomial term, a wrong constant or a broken range
# reduction fails; and the row split is pinned by inputs on which the two
# arms differ.

def _ulp_err(got, x):
    exact = np.exp(x.astype(np.float64))
    spacing = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - exact) / spacing


def test_v_expf_within_the_routines_error_bound():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-87.3, 88.7, 400_000), rng.uniform(-1, 1, 200_000),
                        np.arange(-2000, 2000) * np.float32(np.log(2) / 16)]).astype(np.float32)
    got = O.v_expf(x)
    assert np.max(_ulp_err(got, x)) <= 1.45358 + 0.5
    # and it is not libm's expf (the scalar arm): the two differ on some inputs
    ref = np.array([math.exp(v) for v in x[:2000].astype(np.float64)], np.float32)
    assert np.any(got[:2000] != ref)


def test_v_expf_exact_points_and_range_limits():
    assert O.v_expf(np.array([0.0, -0.0], np.float32)).tolist() == [1.0, 1.0]
    for n in range(-20, 21):  # exp(n ln2) = 2^n within the bound
        x = np.float32(n * math.log(2))
        assert _ulp_err(O.v_expf(np.array([x])), np.array([x]))[0] <= 2.0
    # past the overflow threshold: +inf; far below the subnormals: 0
    big = O.v_expf(np.array([88.73, 89.0, 100.0, 200.0, 1e30], np.float32))
    assert np.all(np.isinf(big)) and np.all(big > 0)
    assert np.all(O.v_expf(np.array([-104.0, -150.0, -1e30], np.float32)) == 0.0)
    # the slow path (|n| > 126) into the subnormals: within a subnormal step
    # plus the relative bound
    x = np.linspace(-103.9, -87.4, 20001).astype(np.float32)
    got = O.v_expf(x).astype(np.float64)
    exact = np.exp(x.astype(np.float64))
    assert np.all(np.abs(got - exact) <= 2.0 ** -149 + 2.5e-7 * exact)
    # near the top of the range (|n| up to 128): finite and within the bound
    x = np.linspace(87.0, 88.72, 20001).astype(np.float32)
    got = O.v_expf(x)
    assert np.all(np.isfinite(got)) and np.max(_ulp_err(got, x)) <= 1.45358 + 0.5


def test_swiglu_rows_take_the_vector_arm_then_the_scalar_tail():
    """Per row of nc: the first nc - nc % 8 elements are v_silu(x) * g, the
    rest the scalar formula.  The inputs are chosen where v_expf and libm's
    expf round differently, so the split is visible."""
    rng = np.random.default_rng(9)
    cand = (rng.standard_normal(20000) * 4).astype(np.float32)
    differ = cand[O.v_expf(-cand) != np.array([np.float32(math.exp(-float(v))) for v in cand], np.float32)]
    vs = np.array([O.lib().orc_v_silu(float(v)) for v in differ], np.float32)
    sc = np.array([np.float32(v) / (np.float32(1.0) + np.float32(math.exp(-float(v)))) for v in differ], np.float32)
    differ = differ[vs != sc]
    assert differ.size >= 64
    for nc in (8, 13, 21, 3):
        rows = 3
        x = differ[:rows * nc].reshape(rows, nc)
        g = np.ones_like(x)
        got = O.glu(O.GLU_SWIGLU, x, g)
        scalar = O.glu_elementwise(O.GLU_SWIGLU, x, g)
        vec = nc - nc % 8
        np.testing.assert_array_equal(got[:, vec:], scalar[:, vec:])
        want_vec = np.array([[O.lib().orc_v_silu(float(v)) for v in row[:vec]] for row in x], np.float32)
        np.testing.assert_array_equal(got[:, :vec], want_vec.reshape(rows, vec))
        if vec:
            assert np.all(got[:, :vec] != scalar[:, :vec])
