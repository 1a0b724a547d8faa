"""The benchmark's memory-rate probes compute what they claim to read and copy:
hb_stream_read's per-wave XOR folds cover every 16-byte word once (their XOR
equals numpy's over the whole buffer, for sizes that end mid-iteration), and
hb_stream_copy reproduces its source, at several launch shapes; so do their
chunked forms."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("words,blocks,nt", [(1, 1, 0), (4097, 3, 1), (1 << 16, 256, 0), ((1 << 20) + 5, 2048, 1)])
def test_stream_read_folds_every_word(bridge, words, blocks, nt):
    from hip_bridge import DeviceBuffer, call, load

    rng = np.random.default_rng(words)
    a = rng.integers(0, 2 ** 32, size=(words, 4), dtype=np.uint64).astype(np.uint32)
    src = DeviceBuffer.from_array(a)
    sink = DeviceBuffer(int(load().hb_stream_read_sink_bytes(blocks)))
    print(f"case: stream read {words} words, {blocks} blocks, nt={nt}", flush=True)
    call("hb_stream_read", src, a.nbytes, sink, blocks, nt, None)
    bridge.synchronize()
    got = np.bitwise_xor.reduce(sink.download(np.uint32, (blocks * 4,)))
    assert got == np.bitwise_xor.reduce(a.reshape(-1))


@pytest.mark.parametrize("words,blocks", [(1, 1), (12345, 7), ((1 << 20) + 3, 1024)])
def test_stream_copy_reproduces_source(bridge, words, blocks):
    from hip_bridge import DeviceBuffer, call

    rng = np.random.default_rng(words + 1)
    a = rng.integers(0, 2 ** 32, size=(words, 4), dtype=np.uint64).astype(np.uint32)
    src, dst = DeviceBuffer.from_array(a), DeviceBuffer(a.nbytes)
    print(f"case: stream copy {words} words, {blocks} blocks", flush=True)
    call("hb_stream_copy", dst, src, a.nbytes, blocks, None)
    bridge.synchronize()
    assert np.array_equal(dst.download(np.uint32, a.shape), a)


@pytest.mark.parametrize("chunks,chunk_kib,nt", [(1, 64, 0), (3, 128, 1), (40, 192, 1)])
def test_chunked_probes(bridge, chunks, chunk_kib, nt):
    """hb_stream_read_chunked folds every word of every chunk once;
    hb_stream_copy_chunked reproduces its source."""
    from hip_bridge import DeviceBuffer, call, load

    chunk = chunk_kib * 1024
    words = chunks * chunk // 16
    rng = np.random.default_rng(chunks * 7 + chunk_kib)
    a = rng.integers(0, 2 ** 32, size=(words, 4), dtype=np.uint64).astype(np.uint32)
    src, dst = DeviceBuffer.from_array(a), DeviceBuffer(a.nbytes)
    sink = DeviceBuffer(int(load().hb_stream_read_sink_bytes(chunks)))
    print(f"case: chunked probes {chunks} x {chunk_kib} KiB, nt={nt}", flush=True)
    call("hb_stream_read_chunked", src, a.nbytes, chunk, sink, nt, None)
    call("hb_stream_copy_chunked", dst, src, a.nbytes, chunk, None)
    bridge.synchronize()
    assert np.bitwise_xor.reduce(sink.download(np.uint32, (chunks * 4,))) == np.bitwise_xor.reduce(a.reshape(-1))
    assert np.array_equal(dst.download(np.uint32, a.shape), a)


def test_probes_refuse_bad_sizes(bridge):
    from hip_bridge import DeviceBuffer, HipBridgeError, call

    buf = DeviceBuffer(64)
    with pytest.raises(HipBridgeError, match="multiple of 16"):
        call("hb_stream_read", buf, 24, buf, 1, 0, None)
    with pytest.raises(HipBridgeError, match="blocks"):
        call("hb_stream_copy", buf, buf, 32, 0, None)
    with pytest.raises(HipBridgeError, match="64 KiB"):
        call("hb_stream_copy_chunked", buf, buf, 64, 64, None)
    with pytest.raises(HipBridgeError, match="chunks"):
        call("hb_stream_read_chunked", buf, 3 << 15, 1 << 16, buf, 0, None)
