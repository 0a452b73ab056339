"""GGUF v3 reader (host side, no GPU): header / metadata / tensor-info parsing
of files written to the reference's documented layout, and rejection of
malformed files with an error before anything is allocated on the device."""
import struct

import numpy as np
import pytest

from gguf_writer import write_gguf


@pytest.fixture(scope="module")
def lx():
    from larynx_amd import gguf
    from larynx_amd._lib import LX_ERR_ARG, LxError
    return gguf, LX_ERR_ARG, LxError


def test_parse_tensors_and_metadata(tmp_path, lx):
    gguf, _, _ = lx
    rng = np.random.default_rng(0)
    tensors = [("input_embedding.weight", rng.standard_normal((7, 80)).astype(np.float32)),
               ("pre_lookahead_layer.conv1.weight",
                rng.standard_normal((16, 80, 4)).astype(np.float32)),
               ("a.bias", np.arange(5, dtype=np.float32)),  # 20 bytes: padded to 32
               ("half", np.ones((3, 3), np.float16)),
               ("ids", np.arange(6, dtype=np.int32).reshape(2, 3)),
               ("d", np.zeros((2, 2, 2, 2), np.float64))]
    p = tmp_path / "t.gguf"
    write_gguf(p, tensors, arch="cosyvoice3.flow", name="unit",
               extra_kv=[("some.array", 9, struct.pack("<iQ", 5, 3) + struct.pack("<3i", 1, 2, 3)),
                         ("some.strings", 9, struct.pack("<iQ", 8, 2) + struct.pack("<Q", 1) + b"x"
                          + struct.pack("<Q", 2) + b"yz"),
                         ("some.f64", 12, struct.pack("<d", 1.5))])
    g = gguf.GgufFile(p, device=False)
    assert g.metadata("general.architecture") == "cosyvoice3.flow"
    assert g.metadata("general.name") == "unit"
    assert g.metadata("absent") is None
    assert len(g) == len(tensors)
    for i, (name, arr) in enumerate(tensors):
        n, typ, shape, nbytes = g.info(i)
        assert n == name and shape == arr.shape and nbytes == arr.nbytes
        assert gguf.GGML_TYPES[typ] == {"float32": "F32", "float16": "F16", "int32": "I32",
                                        "float64": "F64"}[arr.dtype.name]
        assert g.find(name) == i
        assert g.data_ptr(name) is None  # host-only parse: nothing on the device
    assert g.find("missing") == -1
    g.close()


def _bad(tmp_path, data):
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    return p


def test_rejects_malformed_files(tmp_path, lx):
    gguf, ERR_ARG, LxError = lx
    good = tmp_path / "g.gguf"
    write_gguf(good, [("w", np.ones((4, 8), np.float32)), ("b", np.ones(4, np.float32))])
    raw = good.read_bytes()

    def rejects(data, what):
        with pytest.raises(LxError) as e:
            gguf.GgufFile(_bad(tmp_path, data), device=False)
        assert e.value.code == ERR_ARG
        assert what in str(e.value), str(e.value)

    rejects(b"GGML" + raw[4:], "not a GGUF file")
    rejects(raw[:4] + struct.pack("<I", 2) + raw[8:], "version")
    rejects(raw[:10], "counts")
    rejects(raw[:60], "truncated")
    rejects(raw[:-20], "outside the data section")  # last tensor cut short (past its padding)
    # a block-quantised tensor type (Q4_0 = 2) is refused by name
    q = tmp_path / "q.gguf"
    write_gguf(q, [("w", np.ones((4, 32), np.float32))])
    qb = bytearray(q.read_bytes())
    i = qb.find(b"w" + struct.pack("<I", 2))  # name, n_dims
    struct.pack_into("<i", qb, i + 1 + 4 + 16, 2)
    rejects(bytes(qb), "ggml type 2")
    # duplicate names
    d = tmp_path / "d.gguf"
    write_gguf(d, [("w", np.ones(4, np.float32)), ("w", np.ones(4, np.float32))])
    rejects(d.read_bytes(), "duplicate tensor 'w'")
    # absurd string length in the metadata
    rejects(raw[:24] + struct.pack("<Q", 1 << 62) + raw[32:], "truncated metadata")
    with pytest.raises(LxError):
        gguf.GgufFile(tmp_path / "does_not_exist.gguf", device=False)


def test_alignment_from_metadata(tmp_path, lx):
    """general.alignment (u32) replaces the 32-byte default for the data
    section and the tensor offsets."""
    gguf, _, _ = lx
    p = tmp_path / "a.gguf"
    write_gguf(p, [("x", np.ones(3, np.float32)), ("y", np.ones(5, np.float32))],
               extra_kv=[("general.alignment", 4, struct.pack("<I", 64))], align=64)
    g = gguf.GgufFile(p, device=False)
    assert [t[2] for t in g.tensors()] == [(3,), (5,)]
