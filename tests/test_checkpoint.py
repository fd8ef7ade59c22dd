"""Checkpoint formats (host side): the reference's own fixture files (copied data under tests/golden/,
from tensor/safetensors/testdata and tensor/npy/testdata) decoded with the values its tests expect
(tensor/safetensors/safetensors_test.go:56-192, 533-622; tensor/npy/npy_test.go:56-320), the writer's
layout (safetensors.go:75-146) and round trips. numpy (allow_pickle=False) and the safetensors package
read the same files as independent decoders."""
import json
import os
import struct

import numpy as np
import pytest

from anneal_amd import _lib as L
from anneal_amd import checkpoint as ck

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ST = lambda n: os.path.join(GOLD, "safetensors", n)  # noqa: E731
NP = lambda n: os.path.join(GOLD, "npy", n)  # noqa: E731


def f32(*v):
    return np.array(v, np.float32)


@pytest.mark.parametrize("fname,key,shape,want", [
    ("f32_3x4.safetensors", "w", (3, 4), np.arange(12, dtype=np.float32)),
    ("f64_exact.safetensors", "v", (4,), f32(0, 1, 2, 100)),
    ("f16.safetensors", "h", (4,), f32(1.0, 2.0, 0.5, 4.0)),
    ("bf16.safetensors", "b", (4,), f32(1.0, -1.0, 0.5, 2.0)),
    ("with_metadata.safetensors", "weights", (2, 3), np.arange(6, dtype=np.float32)),
])
def test_safetensors_fixtures(fname, key, shape, want):
    t = ck.load_tensors(ST(fname))
    assert t[key].shape == shape
    np.testing.assert_array_equal(t[key].ravel(), want)


def test_safetensors_multi_dtype_fixture():
    t = ck.load_tensors(ST("multi_dtype.safetensors"))
    cases = {"i8": [-5, 0, 10, 127], "u8": [0, 1, 255], "i16": [-32768, 0, 32767], "i32": [1, 2, 3],
             "i64": [10, 20, 30], "bool": [1, 0, 1], "f32": [1, 2, 3]}
    for k, v in cases.items():
        np.testing.assert_array_equal(t[k].ravel(), np.array(v, np.float32), err_msg=k)


def test_safetensors_multi_tensor_fixture():
    t = ck.load_tensors(ST("multi_tensor.safetensors"))
    assert sorted(t) == ["bias", "mask", "weights"]
    np.testing.assert_array_equal(t["weights"], np.arange(6, dtype=np.float32).reshape(2, 3))
    np.testing.assert_array_equal(t["bias"], f32(0.0, 0.5, 1.0))
    np.testing.assert_array_equal(t["mask"], f32(1, 0, 1))


def test_safetensors_int_range_error_names_the_value():
    with pytest.raises(L.AnnealHipError, match="16777217"):
        ck.load_tensors(ST("i64_oor.safetensors"))


def test_safetensors_unsupported_dtype(tmp_path):
    hdr = b'{"v":{"dtype":"F8_E4M3","shape":[2],"data_offsets":[0,2]}}'
    p = tmp_path / "f8.safetensors"
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\x00\x00")
    with pytest.raises(L.AnnealHipError, match="F8_E4M3"):
        ck.load_tensors(str(p))


def test_safetensors_f16_bit_patterns(tmp_path):
    """F16 -> f32 widening of IEEE patterns: ±0, 1, -2, max normal, min normal, min subnormal, ±Inf, NaN."""
    bits = np.array([0x0000, 0x8000, 0x3C00, 0xC000, 0x7BFF, 0x0400, 0x0001, 0x7C00, 0xFC00, 0x7E00], np.uint16)
    hdr = json.dumps({"h": {"dtype": "F16", "shape": [len(bits)], "data_offsets": [0, 2 * len(bits)]}}).encode()
    p = tmp_path / "f16bits.safetensors"
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bits.tobytes())
    got = ck.load_tensors(str(p))["h"]
    want = bits.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got[:-1].view(np.uint32), want[:-1].view(np.uint32))
    assert np.isnan(got[-1])


def test_safetensors_writer_layout_and_round_trip(tmp_path):
    """Names sorted, header {"name":{"dtype":"F32","shape":[..],"data_offsets":[a,b]}} padded to 8 bytes
    with spaces (safetensors.go:75-146), data in name order; re-read by this library and by the
    safetensors package."""
    w = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = f32(0.1, 0.2)
    p = str(tmp_path / "fidelity.safetensors")
    ck.save_safetensors(p, {"weight": w, "bias": b})
    raw = open(p, "rb").read()
    hl = struct.unpack("<Q", raw[:8])[0]
    assert hl % 8 == 0
    header = raw[8:8 + hl].decode()
    assert header.rstrip(" ") == ('{"bias":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
                                  '"weight":{"dtype":"F32","shape":[2,3],"data_offsets":[8,32]}}')
    assert raw[8 + hl:] == b.tobytes() + w.tobytes()
    t = ck.load_tensors(p)
    np.testing.assert_array_equal(t["weight"], w)
    np.testing.assert_array_equal(t["bias"], b)
    try:
        from safetensors.numpy import load_file
    except ImportError:
        pytest.skip("safetensors package not importable")
    t2 = load_file(p)
    np.testing.assert_array_equal(t2["weight"], w)
    np.testing.assert_array_equal(t2["bias"], b)


@pytest.mark.parametrize("fname,shape,want", [
    ("float32_3x4.npy", (3, 4), np.arange(12, dtype=np.float32)),
    ("float64_exact.npy", (4,), f32(0, 1, 2, 100)),
    ("int32_2x3.npy", (2, 3), f32(1, 2, 3, 4, 5, 6)),
    ("int8_1d.npy", (4,), f32(-5, 0, 10, 127)),
    ("uint8_1d.npy", (3,), f32(0, 1, 255)),
    ("bool_1d.npy", (4,), f32(1, 0, 1, 1)),
    ("fortran_2x3.npy", (2, 3), f32(0, 1, 2, 3, 4, 5)),
    ("scalar_f32.npy", (), f32(42.0)),
    ("float32_2x3x4.npy", (2, 3, 4), np.arange(24, dtype=np.float32)),
    ("bigendian_f32.npy", (4,), f32(1, 2, 3, 4)),
])
def test_npy_fixtures(fname, shape, want):
    t = ck.load_tensors(NP(fname))
    (arr,) = t.values()
    assert arr.shape == shape
    np.testing.assert_array_equal(arr.ravel(), want)
    ref = np.load(NP(fname), allow_pickle=False)       # numpy as an independent decoder
    np.testing.assert_array_equal(arr, np.ascontiguousarray(ref).astype(np.float32))


def test_npy_errors():
    with pytest.raises(L.AnnealHipError, match="complex"):
        ck.load_tensors(NP("complex64.npy"))
    with pytest.raises(L.AnnealHipError, match="16777217"):
        ck.load_tensors(NP("int64_oor.npy"))


def test_npz_fixture():
    t = ck.load_tensors(NP("multi.npz"))
    assert sorted(t) == ["bias", "mask", "weights"]
    np.testing.assert_array_equal(t["weights"], np.arange(6, dtype=np.float32).reshape(2, 3))
    np.testing.assert_array_equal(t["bias"], f32(0.0, 0.5, 1.0))
    np.testing.assert_array_equal(t["mask"], f32(1, 0, 1))


def test_missing_file_and_garbage(tmp_path):
    with pytest.raises(L.AnnealHipError):
        ck.load_tensors(str(tmp_path / "nope.safetensors"))
    p = tmp_path / "junk.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(L.AnnealHipError, match="header length"):
        ck.load_tensors(str(p))


def test_npz_compressed_members(tmp_path):
    """np.savez_compressed writes deflated ZIP members; Go's archive/zip (the reference's LoadNPZ,
    tensor/npy/npy.go:51-78) reads them, and so does this reader."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal((7, 5)).astype(np.float32)
    b = np.arange(12, dtype=np.int32).reshape(3, 4)
    p = tmp_path / "c.npz"
    np.savez_compressed(p, a=a, b=b, empty=np.zeros((0, 3), np.float32))
    t = ck.load_tensors(str(p))
    np.testing.assert_array_equal(t["a"], a)
    np.testing.assert_array_equal(t["b"], b.astype(np.float32))
    assert t["empty"].shape == (0, 3)


def _safetensors_with_header(p, header: bytes, data: bytes):
    p.write_bytes(struct.pack("<Q", len(header)) + header + data)


def test_safetensors_json_escapes_in_names(tmp_path):
    """Go's json.Marshal (safetensors.Save) writes <, > and & as \\u003c, \\u003e and \\u0026; names with
    every JSON escape, and a surrogate pair, decode to the same UTF-8 name."""
    data = np.arange(2, dtype=np.float32).tobytes()
    names = {r"a<b&c>": "a<b&c>", r"q\"\\\/\b\f\n\r\t": "q\"\\/\b\f\n\r\t",
             r"é😀": "é\U0001F600"}
    for raw, want in names.items():
        p = tmp_path / "e.safetensors"
        hdr = ('{"%s":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}' % raw).encode()
        _safetensors_with_header(p, hdr, data)
        t = ck.load_tensors(str(p))
        assert list(t) == [want]
        np.testing.assert_array_equal(t[want], [0, 1])


def test_safetensors_writer_escapes_round_trip(tmp_path):
    p = str(tmp_path / "w.safetensors")
    name = "ctl\x01\ttab<&>é"
    ck.save_safetensors(p, {name: np.ones(3, np.float32)})
    assert list(ck.load_tensors(p)) == [name]


@pytest.mark.parametrize("cut", [9, 20, 40, -3])
def test_truncated_files_fail_cleanly(tmp_path, cut):
    """Files cut short anywhere (header length, header, directory) raise an error, never read past the end."""
    src = tmp_path / "full.npz"
    np.savez(src, a=np.arange(6, dtype=np.float32))
    raw = src.read_bytes()
    p = tmp_path / "cut.npz"
    p.write_bytes(raw[:cut])
    with pytest.raises(L.AnnealHipError):
        ck.load_tensors(str(p))
    hdr = b'{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}'
    q = tmp_path / "cut.safetensors"
    full = struct.pack("<Q", len(hdr)) + hdr + np.zeros(2, np.float32).tobytes()
    q.write_bytes(full[:cut])
    with pytest.raises(L.AnnealHipError):
        ck.load_tensors(str(q))


def test_bad_json_escapes_are_errors(tmp_path):
    for raw in (r"bad\x", r"\ud83d", r"\u12"):
        p = tmp_path / "b.safetensors"
        hdr = ('{"%s":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}' % raw).encode()
        _safetensors_with_header(p, hdr, np.zeros(2, np.float32).tobytes())
        with pytest.raises(L.AnnealHipError):
            ck.load_tensors(str(p))
