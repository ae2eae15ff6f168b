"""The safetensors reader behind ixh_model_load_safetensors, on the CPU
(ixh_safetensors_tensor touches no GPU): the reference's own tests
(safetensors/safetensors_test.go) restated with their bytes and values,
plus the checks of entry.bytes (safetensors.go:192-224)."""
import math
import struct

import numpy as np
import pytest

from indecis_amd import _lib
from indecis_amd import safetensors as st


def _raw_file(tmp_path, header, data=b"", name="t.safetensors"):
    p = tmp_path / name
    hb = header.encode() if isinstance(header, str) else header
    p.write_bytes(struct.pack("<Q", len(hb)) + hb + data)
    return p


def test_write_parse_round_trip(tmp_path):
    """TestWriteParseRoundTrip (safetensors_test.go:11-27)."""
    p = tmp_path / "rt.safetensors"
    b = np.array([[1, 2, 3], [4, 5, math.pi]], np.float32)
    a = np.array([-0.5], np.float32)
    st.write(p, {"b": b, "a": a}, {"format": "indecis"})
    assert np.array_equal(st.tensor(p, "b"), b.reshape(-1))
    assert np.array_equal(st.tensor(p, "a"), a)
    raw = p.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    assert n % 8 == 0 and b'"__metadata__":{"format":"indecis"}' in raw[8:8 + n]


def test_parse_bf16_and_f16(tmp_path):
    """TestParseBF16AndF16 (safetensors_test.go:29-50): the same header and
    bytes, the same values (bf16 1, -3; f16 1, -0.5, the smallest
    subnormal)."""
    header = ('{"x":{"dtype":"BF16","shape":[2],"data_offsets":[0,4]},'
              '"y":{"dtype":"F16","shape":[3],"data_offsets":[4,10]}}')
    data = struct.pack("<5H", 0x3F80, 0xC040, 0x3C00, 0xB800, 0x0001)
    p = _raw_file(tmp_path, header, data)
    assert st.tensor(p, "x").tolist() == [1.0, -3.0]
    y = st.tensor(p, "y")
    assert y[0] == 1 and y[1] == -0.5 and abs(float(y[2]) - 5.960464477539063e-08) <= 1e-15


def test_parse_rejects_corruption(tmp_path):
    """TestParseRejectsCorruption (safetensors_test.go:52-68): a short file,
    a giant header, a size that does not match the shape."""
    cases = {
        "short": (tmp_path / "short", bytes([1, 2, 3])),
        "giant header": (tmp_path / "giant", struct.pack("<Q", 1 << 40) + b"{}"),
    }
    header = b'{"x":{"dtype":"F32","shape":[4],"data_offsets":[0,8]}}'
    cases["inconsistent size"] = (tmp_path / "bad", struct.pack("<Q", len(header)) + header + bytes(8))
    msgs = {"short": "truncated file", "giant header": "invalid", "inconsistent size": "8 bytes for 4 F32"}
    for name, (p, raw) in cases.items():
        p.write_bytes(raw)
        with pytest.raises(_lib.IxhError, match=msgs[name]) as e:
            st.tensor(p, "x")
        assert e.value.code == _lib.IXH_EFORMAT, name


def test_write_bf16(tmp_path):
    """TestWriteBF16 (safetensors_test.go:70-83): written in bf16, 1 and
    -2.5 come back exactly, 0.1 within 1e-3 and not exactly."""
    p = tmp_path / "bf.safetensors"
    st.write(p, {"x": (np.array([1, -2.5, 0.1], np.float32), "BF16")})
    got = st.tensor(p, "x")
    assert got[0] == 1 and got[1] == -2.5 and abs(float(got[2]) - 0.1) <= 1e-3 and got[2] != np.float32(0.1)


def test_to_bf16_ties_to_even():
    """ToBF16 (safetensors.go:334-342): nearest, ties to even, NaN kept."""
    v = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5], np.float32)
    assert st.to_bf16(v).tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC020]
    assert (st.to_bf16(np.array([np.nan], np.float32))[0] & 0x7FC0) == 0x7FC0


@pytest.mark.parametrize("header,data,msg", [
    ('{"x":{"dtype":"F64","shape":[1],"data_offsets":[0,8]}}', bytes(8), "unsupported dtype F64"),
    ('{"x":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', bytes(4), "invalid shape"),
    ('{"x":{"dtype":"F32","shape":[2],"data_offsets":[4,12]}}', bytes(8), "out of data bounds"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}}', bytes(8), "out of data bounds"),
    ('{"x":{"dtype":"F32","shape":[1]}}', bytes(4), "dtype, shape and data_offsets"),
    ('{"x":', b"", "object expected"),
    ('{"x":{"dtype":"I8","shape":[2],"data_offsets":[0,2]}} junk', bytes(2), "trailing"),
])
def test_entry_checks(tmp_path, header, data, msg):
    """entry.bytes (safetensors.go:192-224) and the header parse."""
    p = _raw_file(tmp_path, header, data)
    with pytest.raises(_lib.IxhError, match=msg):
        st.tensor(p, "x")


def test_metadata_and_i8(tmp_path):
    """Nested metadata is skipped; I8 decodes to the integers; a missing
    name is an error."""
    header = ('{"__metadata__":{"a":{"b":[1,2,{"c":"d\\"e"}]},"f":"g"},'
              '"q":{"dtype":"I8","shape":[2,2],"data_offsets":[0,4]}}')
    p = _raw_file(tmp_path, header, bytes([1, 255, 128, 127]))
    assert st.tensor(p, "q").tolist() == [1, -1, -128, 127]
    with pytest.raises(_lib.IxhError, match="no such tensor"):
        st.tensor(p, "nope")
