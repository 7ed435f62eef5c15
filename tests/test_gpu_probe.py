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
