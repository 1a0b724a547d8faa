"""The checkpoint header reader behind rs_mlx_weights_load (host only, no GPU):
files written by the safetensors library itself are accepted with the right
tensor count, and malformed headers are refused before any device memory is
touched (the manifest rules of src/serving/weights.rs:236-301: header length
2 B..8 MiB inside the file, dtypes F32/I32/U32/F16/BF16, rank 1..4 with
positive dimensions, offsets spanning exactly the shape inside the payload,
no overlaps, no duplicate keys)."""
import json
import struct

import numpy as np
import pytest

import ckpt


@pytest.fixture(scope="module")
def lib():
    import hip_bridge

    return hip_bridge


def check(path):
    from hip_bridge.session import safetensors_check

    return safetensors_check(path)


def raw(path, header, payload=b"", pad=True):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    if pad:
        h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + payload)
    return path


def test_library_written_files_are_accepted(lib, tmp_path):
    from safetensors.numpy import save_file

    rng = np.random.default_rng(0)
    tensors = {
        "a.weight": rng.integers(0, 2**32, (16, 8), dtype=np.uint32),
        "a.scales": rng.standard_normal((16, 2)).astype(np.float16),
        "norm": rng.standard_normal(64).astype(np.float32),
        "ids": np.arange(6, dtype=np.int32).reshape(1, 2, 3),
        "x.y.z": np.ones((1, 1, 1, 5), np.float32),
    }
    save_file(tensors, str(tmp_path / "lib.safetensors"), metadata={"format": "mlx"})
    assert check(tmp_path / "lib.safetensors") == len(tensors)
    save_file({}, str(tmp_path / "empty.safetensors"))
    assert check(tmp_path / "empty.safetensors") == 0


def test_own_writer_with_bf16_is_accepted(lib, tmp_path):
    t = {"w": ("BF16", np.zeros((3, 4), np.uint16)), "v": ("F32", np.zeros(2, np.float32))}
    ckpt.write_safetensors(tmp_path / "m.safetensors", t, {"k": "v"})
    assert check(tmp_path / "m.safetensors") == 2


def entry(dtype="F32", shape=(2,), offsets=(0, 8)):
    return {"dtype": dtype, "shape": list(shape), "data_offsets": list(offsets)}


BAD_HEADERS = {
    "not an object": [1, 2],
    "unsupported dtype": {"t": entry(dtype="F64", offsets=(0, 16))},
    "rank 0": {"t": entry(shape=(), offsets=(0, 4))},
    "rank 5": {"t": entry(shape=(1, 1, 1, 1, 2))},
    "zero dimension": {"t": entry(shape=(0, 2), offsets=(0, 0))},
    "negative dimension": {"t": entry(shape=(-2,))},
    "fractional dimension": {"t": entry(shape=(2.0,))},
    "offsets short of the shape": {"t": entry(offsets=(0, 4))},
    "offsets reversed": {"t": entry(offsets=(8, 0))},
    "offsets past the payload": {"t": entry(offsets=(8, 16))},
    "overlapping tensors": {"t": entry(), "u": entry(offsets=(4, 12))},
    "extra field": {"t": dict(entry(), extra=1)},
    "missing field": {"t": {"dtype": "F32", "shape": [2]}},
    "dtype not a string": {"t": entry(dtype=0)},
    "metadata not an object": {"__metadata__": [1], "t": entry()},
    "empty name": {"": entry()},
    "tensor not an object": {"t": [1]},
}


@pytest.mark.parametrize("why", sorted(BAD_HEADERS))
def test_malformed_headers_are_refused(lib, tmp_path, why):
    from hip_bridge import HipBridgeError

    path = raw(tmp_path / "bad.safetensors", BAD_HEADERS[why], b"\0" * 12)
    with pytest.raises(HipBridgeError, match="safetensors"):
        check(path)


RAW_BAD = {
    "duplicate key": b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}, '
                     b'"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}',
    "trailing bytes": b'{} {}',
    "truncated JSON": b'{"t": {"dtype": "F32"',
    "unterminated string": b'{"t',
    "bad escape": b'{"\\q": {}}',
    "unpaired surrogate": b'{"\\ud800": {}}',
    "control character": b'{"a\x01": {}}',
    "leading zero": b'{"t": {"dtype": "F32", "shape": [02], "data_offsets": [0, 8]}}',
    "deep nesting": b'{"__metadata__": ' + b'[' * 40 + b']' * 40 + b'}',
    "huge offset": b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 99999999999999999999999]}}',
}


@pytest.mark.parametrize("why", sorted(RAW_BAD))
def test_malformed_json_is_refused(lib, tmp_path, why):
    from hip_bridge import HipBridgeError

    path = raw(tmp_path / "bad.safetensors", RAW_BAD[why], b"\0" * 8)
    with pytest.raises(HipBridgeError, match="safetensors"):
        check(path)


def test_escaped_names_decode(lib, tmp_path):
    h = b'{"caf\\u00e9 \\ud83d\\ude00\\n": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}'
    assert check(raw(tmp_path / "esc.safetensors", h, b"\0" * 8)) == 1


def test_file_level_refusals(lib, tmp_path):
    from hip_bridge import HipBridgeError

    cases = {
        "short.safetensors": b"\x02\0\0",
        "len1.safetensors": struct.pack("<Q", 1) + b"{",
        "past_end.safetensors": struct.pack("<Q", 64) + b"{}",
        "huge.safetensors": struct.pack("<Q", 9 << 20) + b"{}",
    }
    for name, data in cases.items():
        (tmp_path / name).write_bytes(data)
        with pytest.raises(HipBridgeError, match="safetensors"):
            check(tmp_path / name)
    with pytest.raises(HipBridgeError, match="not a regular file"):
        check(tmp_path)
    with pytest.raises(HipBridgeError, match="cannot stat"):
        check(tmp_path / "absent.safetensors")
    (tmp_path / "link.safetensors").symlink_to(tmp_path / "len1.safetensors")
    with pytest.raises(HipBridgeError, match="not a regular file"):
        check(tmp_path / "link.safetensors")


def test_store_rules_before_device_use(lib, tmp_path):
    """A synthetic store takes no checkpoint, and a malformed file loads nothing."""
    from hip_bridge import HipBridgeError
    from hip_bridge.session import WeightStore

    good = raw(tmp_path / "g.safetensors", {"t": entry()}, b"\0" * 8)
    syn = WeightStore(7, 0)
    with pytest.raises(HipBridgeError, match="synthetic"):
        syn.load(good)
    s = WeightStore()
    with pytest.raises(HipBridgeError, match="safetensors"):
        s.load(raw(tmp_path / "b.safetensors", {"t": entry(offsets=(0, 4))}, b"\0" * 8))
