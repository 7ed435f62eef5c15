"""Input generators of the reference's golden tests, restated in numpy float32.

quant_src / quant_imatrix: src/ggml/quants/testing.zig:33-89 (the LCG of
harness/quants_golden.c, five patterns, 4 rows x 256).
vecdot_fill: src/ggml/cpu/quants/testing.zig:86-132 (the LCG of
harness/vecdot_golden.c, six patterns, 512 elements).
Every operation is a float32 operation in the order the reference writes it.
"""
import numpy as np

F = np.float32
QUANT_PATTERNS = ("random", "zeros", "constant", "outlier", "alternating")
VECDOT_PATTERNS = ("random", "zeros", "signs", "opposed", "lopsided", "ties")


class _QuantRng:
    def __init__(self, state):
        self.state = state

    def next(self):
        self.state = (self.state * 1664525 + 1013904223) & 0xFFFFFFFF
        v = F(self.state >> 8) / F(1 << 24)
        return F(v * F(4.0) - F(2.0))


def quant_src(pattern, n_rows=4, n_per_row=256):
    n = n_rows * n_per_row
    src = np.zeros(n, dtype=F)
    if pattern == "zeros":
        pass
    elif pattern == "constant":
        src[:] = F(0.5)
    elif pattern == "outlier":
        src[:] = F(0.001)
        for r in range(n_rows):
            src[r * n_per_row + 7] = F(100.0)
    elif pattern == "alternating":
        src[:] = np.where(np.arange(n) & 1, F(-1.25), F(1.25))
    elif pattern == "random":
        rng = _QuantRng(12345)
        for i in range(n):
            src[i] = rng.next()
    else:
        raise ValueError(pattern)
    return src


def quant_imatrix(n_per_row=256):
    rng = _QuantRng(999)
    out = np.zeros(n_per_row, dtype=F)
    for i in range(n_per_row):
        out[i] = F(F(rng.next() + F(2.0)) * F(0.5)) + F(0.01)
    return out


class _VecdotLcg:
    def __init__(self):
        self.state = 1

    def next(self):
        self.state = (1103515245 * self.state + 12345) & 0xFFFFFFFF
        return F(F(self.state >> 16) / F(32768.0)) - F(1.0)


def vecdot_fill(pattern, nelem=512):
    x = np.zeros(nelem, dtype=F)
    y = np.zeros(nelem, dtype=F)
    lcg = _VecdotLcg()
    for i in range(nelem):
        if pattern == "random":
            x[i] = lcg.next()
            y[i] = lcg.next()
        elif pattern == "zeros":
            pass
        elif pattern == "signs":
            x[i] = F(1.0) if i % 2 else F(-0.5)
            y[i] = F(0.75) if i % 3 else F(-1.0)
        elif pattern == "opposed":
            x[i] = lcg.next()
            y[i] = -x[i]
        elif pattern == "lopsided":
            x[i] = lcg.next() * F(1e-4)
            y[i] = lcg.next() * F(4.0)
        elif pattern == "ties":
            if i == 0:
                x[i] = y[i] = F(127.0)
            else:
                half = F(i % 9 - 4) + F(0.5)
                x[i] = half
                y[i] = -half
        else:
            raise ValueError(pattern)
    return x, y
