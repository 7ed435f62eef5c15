"""The streaming-read probe the GEMV's floor is measured with: every byte is
read (the sink holds the XOR of each wave's loads, checked against numpy),
including a ragged last workgroup."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 32768, 1 << 20, (1 << 20) + 4112])
def test_probe_reads_every_byte(nbytes):
    import ggml_hip as G
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    sink = G.probe_stream_read(torch.from_numpy(host.view(np.int32)).cuda()).cpu().numpy().view(np.uint32)
    per_wg = 256 * 8 * 4  # uint32 words per workgroup
    nb = -(-host.size // per_wg)
    pad = np.zeros(nb * per_wg, dtype=np.uint32)
    pad[:host.size] = host
    # [workgroup, load u, wave, lane, word]: thread (wave, lane) loads uint4 index 256 u + 64 wave + lane
    want = np.bitwise_xor.reduce(pad.reshape(nb, 8, 4, 64, 4), axis=(1, 3, 4)).reshape(-1)
    assert sink.size == want.size
    np.testing.assert_array_equal(sink, want)


def test_mfma_valu_probe_does_its_work():
    """Each mode of the overlap probe does the work it is timed for: the MFMA sums
    of mode 3 equal mode 1's and its FMA sums mode 2's, bit for bit; mode 4 splits
    them by wave; a mode without MFMAs leaves zeros and one without FMAs the
    start values."""
    import ggml_hip as G
    nb, iters = 8, 50
    n = nb * 256
    r = {m: G.probe_mfma_valu(m, iters, nb).cpu().numpy() for m in (1, 2, 3, 4)}
    mf, fm = (lambda a: a[:n]), (lambda a: a[n:])
    lane = np.arange(n) % 64
    start = np.float32(16 * 2) * lane + np.float32(2 * sum(range(16)))  # sum of the untouched FMA registers
    assert np.all(np.isfinite(r[3])) and np.any(mf(r[1]) != 0)
    np.testing.assert_array_equal(mf(r[3]), mf(r[1]))
    np.testing.assert_array_equal(fm(r[3]), fm(r[2]))
    np.testing.assert_array_equal(mf(r[2]), np.zeros(n, np.float32))
    np.testing.assert_allclose(fm(r[1]), start, rtol=1e-6)
    even = ((np.arange(n) // 64) % 2) == 0
    np.testing.assert_array_equal(mf(r[4])[even], mf(r[1])[even])
    np.testing.assert_array_equal(fm(r[4])[~even], fm(r[2])[~even])
