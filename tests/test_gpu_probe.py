"""The measurement probes bench.py times (libqmm_probe.so, built from
llama.zig_amd/probes/probe.hip, apart from the backend library):

- the streaming-read probe the GEMV's floor is measured with reads every byte
  (the sink holds the XOR of each wave's loads, checked against numpy),
  including a ragged last workgroup;
- the headline GEMV's access-pattern probe loads exactly the GEMV's bytes
  (per wave: each lane's 16-byte block header and its two 16-byte nibble
  chunks of two rows, XOR-folded), rows past the end clamped to the last;
- each mode of the MFMA / VALU overlap probe does the work it is timed for."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 32768, 1 << 20, (1 << 20) + 4112])
def test_probe_reads_every_byte(nbytes):
    from ggml_hip import probes as P
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    sink = P.stream_read(torch.from_numpy(host.view(np.int32)).cuda()).cpu().numpy().view(np.uint32)
    per_wg = 256 * 8 * 4  # uint32 words per workgroup
    nb = -(-host.size // per_wg)
    pad = np.zeros(nb * per_wg, dtype=np.uint32)
    pad[:host.size] = host
    # [workgroup, load u, wave, lane, word]: thread (wave, lane) loads uint4 index 256 u + 64 wave + lane
    want = np.bitwise_xor.reduce(pad.reshape(nb, 8, 4, 64, 4), axis=(1, 3, 4)).reshape(-1)
    assert sink.size == want.size
    np.testing.assert_array_equal(sink, want)


@pytest.mark.parametrize("nrows", [28, 100, 14336])
def test_gemv_pattern_probe_loads_the_gemv_bytes(nrows):
    from ggml_hip import probes as P
    rng = np.random.default_rng(nrows)
    w = rng.integers(0, 256, size=(nrows, 2304), dtype=np.uint8)
    nwaves = -(-nrows // 28) * 14
    sink = torch.zeros(nwaves, dtype=torch.int32, device="cuda")
    P.q4k_gemv_pattern(torch.from_numpy(w).cuda(), sink)
    got = sink.cpu().numpy().view(np.uint32)
    words = w.view(np.uint32).reshape(nrows, 16, 36)  # [row, super-block, word of the 144 bytes]
    want = np.zeros(nwaves, dtype=np.uint32)
    for wv in range(nwaves):
        v = np.uint32(0)
        for r in range(2):
            row = min(2 * wv + r, nrows - 1)
            for c in range(4):  # the four lanes of each super-block: header + nibble chunks 32c .. 32c + 32
                sel = np.r_[0:4, 4 + 8 * c:12 + 8 * c]
                v ^= np.bitwise_xor.reduce(words[row][:, sel].reshape(-1))
        want[wv] = v
    np.testing.assert_array_equal(got, want)


def test_mfma_valu_probe_does_its_work():
    """Modes 3 and 5 (both kinds in every wave) give every thread mode 1's MFMA
    sums and mode 2's FMA sums, bit for bit.  Modes 4 and 6 run the MFMAs only
    in waves 0-3 and the FMAs only in waves 4-7, each twice as many: their
    MFMA sums there equal a two-iteration-per-step chain (mode 1 at 2 x iters),
    the other half keeps its start values, so neither half ran the other's
    work.  The HW_ID words name one CU per workgroup and SIMDs 0-3."""
    from ggml_hip import probes as P
    nb, iters = 8, 50
    n = nb * P.OV_THREADS
    r = {m: [t.cpu().numpy() for t in P.mfma_valu(m, iters, nb)] for m in P.OV_MODES}
    r2 = [t.cpu().numpy() for t in P.mfma_valu(1, 2 * iters, nb)]
    r2f = [t.cpu().numpy() for t in P.mfma_valu(2, 2 * iters, nb)]
    mf, fm = (lambda a: a[:n]), (lambda a: a[n:])
    lane = np.arange(n) % 64
    start = np.float32(16 * 2) * lane + np.float32(2 * sum(range(16)))  # sum of the untouched FMA registers
    assert np.all(np.isfinite(r[3][0])) and np.any(mf(r[1][0]) != 0)
    for m in (3, 5):
        np.testing.assert_array_equal(mf(r[m][0]), mf(r[1][0]))
        np.testing.assert_array_equal(fm(r[m][0]), fm(r[2][0]))
    np.testing.assert_array_equal(mf(r[2][0]), np.zeros(n, np.float32))
    np.testing.assert_allclose(fm(r[1][0]), start, rtol=1e-6)
    first = ((np.arange(n) // 64) % 8) < 4
    for m in (4, 6):
        np.testing.assert_array_equal(mf(r[m][0])[first], mf(r2[0])[first])
        np.testing.assert_array_equal(mf(r[m][0])[~first], np.zeros(int((~first).sum()), np.float32))
        np.testing.assert_array_equal(fm(r[m][0])[~first], fm(r2f[0])[~first])
        np.testing.assert_allclose(fm(r[m][0])[first], start[first], rtol=1e-6)
    ids = r[4][1].astype(np.int64).reshape(nb, 8)
    assert np.all(((ids >> 4) & 3) < 4)
    cu = (ids >> 8) & 15
    assert np.all(cu == cu[:, :1])
