"""safetensors header parsing through the C-ABI (host only, no GPU):
files written by the official `safetensors` package (an independent
writer), and the malformed files the reference's loader rejects
(model/safetensors.go:63-128: bad header length, bad JSON, unsupported
dtype) plus the offset and size checks of the safetensors format."""
import json
import struct

import numpy as np
import pytest

from gorch_amd import hip


def write_raw(path, header: dict, data: bytes, header_len=None):
    hj = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj) if header_len is None else header_len))
        f.write(hj)
        f.write(data)


def test_names_shapes_dtypes_from_reference_writer(tmp_path):
    import safetensors.numpy
    import safetensors.torch
    import torch

    p1 = tmp_path / "np.safetensors"
    safetensors.numpy.save_file({"weight": np.arange(6, dtype=np.float32).reshape(2, 3),
                                 "bias": np.array([0.1, 0.2, 0.3], np.float32),
                                 "half": np.ones((4, 1, 2), np.float16),
                                 "scalar": np.array(7.0, np.float32),
                                 "empty": np.zeros((0, 5), np.float32)},
                                str(p1), metadata={"format": "np", "note": "a \"quoted\" value"})
    st = hip.SafeTensors(str(p1))
    assert st.names() == sorted(["weight", "bias", "half", "scalar", "empty"])
    assert st.info("weight") == ("F32", (2, 3), 24)
    assert st.info("bias") == ("F32", (3,), 12)
    assert st.info("half") == ("F16", (4, 1, 2), 16)
    assert st.info("scalar") == ("F32", (), 4)
    assert st.info("empty") == ("F32", (0, 5), 0)
    with pytest.raises(hip.HipError):
        st.info("missing")
    st.close()

    p2 = tmp_path / "bf16.safetensors"
    safetensors.torch.save_file({"w_bf16": torch.zeros((2, 3), dtype=torch.bfloat16),
                                 "w_f32": torch.zeros(4)}, str(p2))
    st = hip.SafeTensors(str(p2))
    assert st.names() == ["w_bf16", "w_f32"]
    assert st.info("w_bf16") == ("BF16", (2, 3), 12)
    st.close()


@pytest.mark.parametrize("case", ["short", "hlen", "json", "dtype", "offsets", "size", "dup", "missing_key"])
def test_rejects_malformed(tmp_path, case):
    p = tmp_path / f"{case}.safetensors"
    good = {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "hlen":
        write_raw(p, good, b"\0" * 8, header_len=1 << 20)
    elif case == "json":
        hj = b'{"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]'
        p.write_bytes(struct.pack("<Q", len(hj)) + hj + b"\0" * 8)
    elif case == "dtype":   # the reference: unsupported dtype "I64" for tensor "t"
        write_raw(p, {"t": {"dtype": "I64", "shape": [1], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "offsets":
        write_raw(p, {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4)
    elif case == "size":
        write_raw(p, {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, b"\0" * 8)
    elif case == "dup":
        hj = b'{"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, ' \
             b'"t": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}'
        p.write_bytes(struct.pack("<Q", len(hj)) + hj + b"\0" * 8)
    elif case == "missing_key":
        write_raw(p, {"t": {"dtype": "F32", "shape": [2]}}, b"\0" * 8)
    with pytest.raises(hip.HipError) as e:
        hip.SafeTensors(str(p))
    if case == "dtype":
        assert 'unsupported dtype "I64" for tensor "t"' in str(e.value)


def test_missing_file():
    with pytest.raises(hip.HipError):
        hip.SafeTensors("/nonexistent/model.safetensors")
