"""Checkpoint files in the reference's format (include/inferno/checkpoint/checkpoint.h:5-26,
src/inferno/checkpoint/checkpoint.cpp): written by the C++ layer and parsed here field by
field, written here and loaded by the C++ layer, on the CPU device (and through a HIP module
with -m gpu).

Layout pinned (packed, little-endian): header = magic char[8] "INFERNO\\0", uint32 version (0),
uint32 tensor_count; per tensor: uint32 name_length, uint32 dtype (the raw DType value:
Float32 = 0 ... BFloat16 = 6), uint32 ndim, uint64 numel, uint64 nbytes, ndim x uint64 dims,
the name bytes, nbytes of element data; tensors in state-dict (name) order.
"""
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "cpp" / "api_driver"

# The CkptNet of api_driver.cpp: name -> (dtype code, shape)
NET = {
    "emb.weight": (0, (5, 4)), "fc.bias": (0, (3,)), "fc.weights": (0, (4, 3)), "half.bias": (6, (2,)),
    "half.weights": (6, (2, 2)), "norm.beta": (0, (3,)), "norm.gamma": (0, (3,)),
}


def run(*args):
    if not DRIVER.exists():
        pytest.skip("api_driver not built")
    return subprocess.run([str(DRIVER), *map(str, args)], capture_output=True, text=True, timeout=300)


def parse_printed(out):
    d = {}
    for line in out.strip().splitlines():
        parts = line.split()
        d[parts[0]] = (parts[1], np.array([float(x) for x in parts[2:]]))
    return d


def parse_file(path):
    b = Path(path).read_bytes()
    magic, version, count = struct.unpack_from("<8sII", b, 0)
    off = 16
    recs = []
    for _ in range(count):
        name_len, dtype, ndim, numel, nbytes = struct.unpack_from("<IIIQQ", b, off)
        off += 28
        dims = struct.unpack_from(f"<{ndim}Q", b, off)
        off += 8 * ndim
        name = b[off:off + name_len].decode()
        off += name_len
        data = b[off:off + nbytes]
        off += nbytes
        recs.append((name, dtype, dims, numel, nbytes, data))
    assert off == len(b)
    return magic, version, recs


def decode(dtype, data):
    if dtype == 0:
        return np.frombuffer(data, "<f4").astype(np.float64)
    assert dtype == 6
    return (np.frombuffer(data, "<u2").astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def write_file(path, tensors):
    out = bytearray(struct.pack("<8sII", b"INFERNO\0", 0, len(tensors)))
    for name, (dtype, shape, values) in tensors.items():
        v = np.asarray(values, np.float32).reshape(shape)
        data = v.tobytes() if dtype == 0 else (v.view(np.uint32) >> 16).astype("<u2").tobytes()
        out += struct.pack("<IIIQQ", len(name), dtype, len(shape), v.size, len(data))
        out += struct.pack(f"<{len(shape)}Q", *shape)
        out += name.encode() + data
    Path(path).write_bytes(bytes(out))


def test_saved_file_has_the_reference_layout(tmp_path):
    f = tmp_path / "net.ckpt"
    r = run("ckpt-save", f, "cpu")
    assert r.returncode == 0, r.stderr
    printed = parse_printed(r.stdout)
    magic, version, recs = parse_file(f)
    assert magic == b"INFERNO\0" and version == 0
    assert [x[0] for x in recs] == sorted(NET)
    for name, dtype, dims, numel, nbytes, data in recs:
        code, shape = NET[name]
        assert (dtype, dims) == (code, shape), name
        assert numel == int(np.prod(shape)) and nbytes == numel * (4 if code == 0 else 2)
        np.testing.assert_allclose(decode(dtype, data), printed[name][1], rtol=1e-5, atol=1e-6)


def test_python_written_file_loads_exactly(tmp_path):
    f = tmp_path / "py.ckpt"
    tensors = {n: (c, s, (np.arange(int(np.prod(s))) - 3) / 8.0) for n, (c, s) in NET.items()}
    write_file(f, tensors)
    r = run("ckpt-load", f, "cpu")
    assert r.returncode == 0, r.stderr
    got = parse_printed(r.stdout)
    for n, (c, s, v) in tensors.items():
        assert np.array_equal(got[n][1], v), n


def test_round_trip_and_errors(tmp_path):
    f = tmp_path / "net.ckpt"
    saved = parse_printed(run("ckpt-save", f, "cpu").stdout)
    loaded = parse_printed(run("ckpt-load", f, "cpu").stdout)
    for n in NET:
        assert np.array_equal(saved[n][1], loaded[n][1]), n
    bad = tmp_path / "bad.ckpt"
    b = bytearray(f.read_bytes())
    b[0:8] = b"INFERNX\0"
    bad.write_bytes(bytes(b))
    r = run("ckpt-load", bad, "cpu")
    assert r.returncode != 0 and "not an Inferno checkpoint" in r.stderr
    # a checkpoint missing one of the module's tensors is refused (strict load)
    part = tmp_path / "part.ckpt"
    write_file(part, {n: (c, s, np.zeros(int(np.prod(s)))) for n, (c, s) in NET.items() if n != "fc.bias"})
    r = run("ckpt-load", part, "cpu")
    assert r.returncode != 0 and "missing" in r.stderr


@pytest.mark.gpu
def test_round_trip_through_hip(tmp_path):
    f = tmp_path / "hip.ckpt"
    r = run("ckpt-save", f, "hip")
    assert r.returncode == 0, r.stderr
    saved = parse_printed(r.stdout)
    for dev in ("cpu", "hip"):
        r2 = run("ckpt-load", f, dev)
        assert r2.returncode == 0, r2.stderr
        got = parse_printed(r2.stdout)
        for n in NET:
            assert np.array_equal(saved[n][1], got[n][1]), (dev, n)


def test_save_replaces_the_file_whole(tmp_path):
    """save() writes a sibling temporary file and renames it over the target: an existing file
    is replaced, and no temporary file is left behind."""
    f = tmp_path / "net.ckpt"
    f.write_bytes(b"an older file")
    r = run("ckpt-save", f, "cpu")
    assert r.returncode == 0, r.stderr
    assert parse_file(f)[0] == b"INFERNO\0"
    assert sorted(p.name for p in tmp_path.iterdir()) == ["net.ckpt"]


def _record_offsets(b):
    """(offset of each record's header, offset past its data) of a well-formed file."""
    off, out = 16, []
    for _ in range(struct.unpack_from("<I", b, 12)[0]):
        name_len, _, ndim, _, nbytes = struct.unpack_from("<IIIQQ", b, off)
        end = off + 28 + 8 * ndim + name_len + nbytes
        out.append((off, end))
        off = end
    return out


@pytest.mark.parametrize("damage,message", [
    ("truncate", "data runs past the end of the file"),
    ("trailing", "bytes follow the last"),
    ("numel", "elements but its dims hold"),
    ("nbytes", "data bytes for"),
    ("dtype", "unknown dtype code 5"),
    ("version", "format version 3 is not supported"),
    ("count", "file ends inside record 7 of 8"),
])
def test_malformed_files_are_refused(tmp_path, damage, message):
    """Each field of the layout is checked on load, with the record and byte offset named."""
    f = tmp_path / "net.ckpt"
    assert run("ckpt-save", f, "cpu").returncode == 0
    b = bytearray(f.read_bytes())
    first = _record_offsets(b)[0][0]
    if damage == "truncate":
        b = b[:-1]
    elif damage == "trailing":
        b += b"\0\0\0"
    elif damage == "numel":
        struct.pack_into("<Q", b, first + 12, struct.unpack_from("<Q", b, first + 12)[0] + 1)
    elif damage == "nbytes":
        struct.pack_into("<Q", b, first + 20, struct.unpack_from("<Q", b, first + 20)[0] - 4)
    elif damage == "dtype":
        struct.pack_into("<I", b, first + 4, 5)  # DType::Invalid
    elif damage == "version":
        struct.pack_into("<I", b, 8, 3)
    elif damage == "count":
        struct.pack_into("<I", b, 12, len(NET) + 1)
    bad = tmp_path / "bad.ckpt"
    bad.write_bytes(bytes(b))
    r = run("ckpt-load", bad, "cpu")
    assert r.returncode != 0 and message in r.stderr, r.stderr
    assert "at byte" in r.stderr
