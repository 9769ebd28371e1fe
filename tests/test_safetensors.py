"""CPU checks of the safetensors reader and weight store (include/h3_safetensors.h,
include/h3_weights.h; reference h3_safetensors.c, h3_weights.c): files written
by the `safetensors` package (an independent implementation of the format)
must parse to the same names, dtypes, shapes and bytes, and malformed files
must be rejected with a reason. Host code only, no GPU calls."""
import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

DTYPES = ["UNKNOWN", "BOOL", "I8", "U8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32",
          "I64", "U64", "F64"]


def raw_file(path, header, payload=b"", length=None):
    """header: dict or bytes, written as the 8-byte little-endian length +
    JSON + payload (length overrides the stored header length)."""
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb) if length is None else length) + hb + payload)


def read_header(qd, path):
    h = qd.StHeader()
    err = C.create_string_buffer(512)
    ok = qd.lib().h3_st_read_header(str(path).encode(), C.byref(h), err, 512)
    return ok, h, err.value.decode()


def tensors_of(h):
    return {h.tensors[i].name.decode(): h.tensors[i] for i in range(h.tensor_count)}


def test_dtype_table(qd):
    L = qd.lib()
    sizes = {"BOOL": 1, "I8": 1, "U8": 1, "I16": 2, "U16": 2, "F16": 2, "BF16": 2, "I32": 4,
             "U32": 4, "F32": 4, "I64": 8, "U64": 8, "F64": 8}
    for code, name in enumerate(DTYPES):
        assert L.h3_dtype_name(code).decode() == name
        assert L.h3_dtype_size(code) == sizes.get(name, 0)


def test_reads_files_written_by_safetensors(qd, tmp_path):
    """safetensors.torch.save_file output (bf16, f32, i8, a scalar, metadata):
    every tensor's dtype, shape, byte range and payload round-trip."""
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(3)
    tensors = {
        "transformer_blocks.0.attn.to_q.weight": torch.randn(48, 32, generator=g).bfloat16(),
        "norm.weight": torch.randn(32, generator=g),
        "q8": torch.randint(-127, 128, (5, 7, 3), generator=g, dtype=torch.int8),
        "scalar": torch.tensor(2.5, dtype=torch.float64),
        "café \"quoted\"": torch.arange(6, dtype=torch.int32).reshape(2, 3),
    }
    path = tmp_path / "a.safetensors"
    st.save_file(tensors, str(path), metadata={"format": "pt", "note": "{not a tensor}"})
    ok, h, err = read_header(qd, path)
    assert ok, err
    try:
        assert h.file_size == os.path.getsize(path)
        got = tensors_of(h)
        assert sorted(got) == sorted(tensors)
        L = qd.lib()
        for name, t in tensors.items():
            e = got[name]
            want_dt = {torch.bfloat16: "BF16", torch.float32: "F32", torch.int8: "I8",
                       torch.float64: "F64", torch.int32: "I32"}[t.dtype]
            assert DTYPES[e.dtype] == want_dt
            assert [e.shape[i] for i in range(e.ndim)] == list(t.shape)
            assert L.h3_st_tensor_elements(C.byref(e)) == t.numel()
            assert e.file_offset == 8 + h.header_size + e.data_begin
            buf = (C.c_char * (e.data_end - e.data_begin))()
            assert L.h3_st_read_data(C.byref(h), C.byref(e), buf, len(buf), None, 0)
            want = t.contiguous().view(torch.uint8).numpy().tobytes() if t.dim() else \
                t.reshape(1).view(torch.uint8).numpy().tobytes()
            assert bytes(buf) == want, name
            # a read of the wrong size is refused
            err = C.create_string_buffer(256)
            assert not L.h3_st_read_data(C.byref(h), C.byref(e), buf, len(buf) + 1, err, 256)
            assert b"expected" in err.value
        assert L.h3_st_find(C.byref(h), b"missing") is None
        assert L.h3_st_find(C.byref(h), b"q8") is not None
    finally:
        qd.lib().h3_st_free_header(C.byref(h))


BAD = {
    "short file": (None, b"abc"),
    "length beyond file": ({"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, 999),
    "not an object": (b"[1, 2]", None),
    "unterminated": (b'{"a": {"dtype": "F32"', None),
    "unknown dtype": ({"a": {"dtype": "F8_Q", "shape": [1], "data_offsets": [0, 1]}}, None),
    "offsets outside payload": ({"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}},
                                None),
    "size mismatch": ({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 4]}}, None),
    "reversed offsets": ({"a": {"dtype": "U8", "shape": [0], "data_offsets": [4, 0]}}, None),
    "missing shape": ({"a": {"dtype": "F32", "data_offsets": [0, 4]}}, None),
    "negative dim": (b'{"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}', None),
    "fractional dim": (b'{"a": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}', None),
    "nine dims": ({"a": {"dtype": "U8", "shape": [1] * 9, "data_offsets": [0, 1]}}, None),
    "duplicate name": (b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                       b'"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}', None),
    "trailing bytes": (b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}} x', None),
    "nesting bomb": (b'{"__metadata__": ' + b"[" * 200 + b"]" * 200 + b"}", None),
    "bad escape": (b'{"a\\q": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', None),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_rejects_malformed_headers(qd, tmp_path, case):
    header, extra = BAD[case]
    path = tmp_path / "bad.safetensors"
    if header is None:
        path.write_bytes(extra)
    else:
        length = extra if isinstance(extra, int) else None
        raw_file(path, header, b"\0" * 8, length=length)
    ok, h, err = read_header(qd, path)
    assert not ok and err, case
    assert h.tensor_count == 0 and not h.tensors  # nothing left allocated


def test_accepts_spec_edge_cases(qd, tmp_path):
    """Empty tensors, zero-size payload, whitespace padding (the format pads
    the header with spaces to 8 bytes), metadata of any JSON shape."""
    header = (b'{"__metadata__": {"k": [1, -2.5e3, true, null, {"x": "y"}]}, '
              b'"empty": {"dtype": "F32", "shape": [0, 3], "data_offsets": [0, 0]}, '
              b'"one": {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]}}   ')
    path = tmp_path / "edge.safetensors"
    raw_file(path, header, b"\x80\x3f")
    ok, h, err = read_header(qd, path)
    assert ok, err
    got = tensors_of(h)
    assert sorted(got) == ["empty", "one"]
    assert qd.lib().h3_st_tensor_elements(C.byref(got["empty"])) == 0
    qd.lib().h3_st_free_header(C.byref(h))


def test_weight_store_directory(qd, tmp_path):
    """Shards are every *.safetensors file in the directory (other files are
    ignored); a name must be unique across shards; an empty directory fails."""
    st = pytest.importorskip("safetensors.numpy")
    L = qd.lib()
    err = C.create_string_buffer(512)
    assert not L.h3_weight_store_open(str(tmp_path).encode(), err, 512)
    assert b"no safetensors" in err.value
    st.save_file({"a": np.arange(4, dtype=np.float32)}, str(tmp_path / "model-00001.safetensors"))
    st.save_file({"b": np.ones((2, 2), np.int8)}, str(tmp_path / "model-00002.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text("{}")
    s = L.h3_weight_store_open(str(tmp_path).encode(), err, 512)
    assert s, err.value
    try:
        assert L.h3_weight_store_shards(s) == 2
        hp = C.c_void_p()
        ta = L.h3_weight_find(s, b"a", C.byref(hp))
        tb = L.h3_weight_find(s, b"b", None)
        assert ta and tb and hp.value
        assert C.cast(hp, C.POINTER(qd.StHeader)).contents.path.decode().endswith("00001.safetensors")
        assert not L.h3_weight_find(s, b"c", None)
    finally:
        L.h3_weight_store_free(s)
    st.save_file({"a": np.zeros(4, np.float32)}, str(tmp_path / "model-00003.safetensors"))
    assert not L.h3_weight_store_open(str(tmp_path).encode(), err, 512)
    assert b"tensor a is in" in err.value
