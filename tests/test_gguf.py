"""GGUF reader (vinf_3080ti_amd/gguf.py) on files written by tests/gguf_writer.py: the checks of the
reference's engine/tests/test_phase5_gguf.py (tiny file metadata and tensor directory, quantized tensor
sizes and mmap, bad magic) plus every metadata value type, alignment, and malformed files."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from gguf_writer import write_gguf
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd.gguf import GGUFValueType as V, UnsupportedModelError, load_gguf


def test_tiny_f16_metadata_and_tensor_directory(tmp_path):
    p = tmp_path / "tiny.gguf"
    meta = [("general.architecture", V.STRING, "llama"), ("llama.block_count", V.UINT32, 1),
            ("llama.embedding_length", V.UINT32, 8),
            ("tokenizer.ggml.tokens", V.ARRAY, (V.STRING, [str(i) for i in range(8)]))]
    offs = write_gguf(p, meta, [("token_embd.weight", (8, 8), T.F16, bytes(8 * 8 * 2))])
    g = load_gguf(p)
    assert g.version == 3 and g.alignment == 32 and g.data_start % 32 == 0
    assert g.metadata_value("general.architecture") == "llama"
    assert g.metadata["llama.block_count"].type is V.UINT32
    assert g.metadata_value("tokenizer.ggml.tokens") == [str(i) for i in range(8)]
    assert g.metadata_value("missing", 7) == 7
    t = g.tensors["token_embd.weight"]
    assert t.dimensions == (8, 8) and t.tensor_type is T.F16 and not t.is_quantized
    assert t.numel == 64 and t.nbytes == 128 and t.absolute_offset == offs[0] == g.data_start
    assert g.quantized_tensors() == []


def test_every_metadata_value_type_and_version_2(tmp_path):
    p = tmp_path / "meta.gguf"
    meta = [("u8", V.UINT8, 250), ("i8", V.INT8, -7), ("u16", V.UINT16, 65000), ("i16", V.INT16, -30000),
            ("u32", V.UINT32, 4_000_000_000), ("i32", V.INT32, -2_000_000_000), ("f32", V.FLOAT32, 0.5),
            ("b", V.BOOL, True), ("s", V.STRING, "héllo"), ("u64", V.UINT64, 2**63 + 5),
            ("i64", V.INT64, -(2**62)), ("f64", V.FLOAT64, -1.25e-300),
            ("nested", V.ARRAY, (V.ARRAY, [(V.INT32, [1, -2]), (V.INT32, [])]))]
    write_gguf(p, meta, [], version=2)
    g = load_gguf(p)
    assert g.version == 2 and g.tensors == {}
    for key, vt, value in meta[:-1]:
        assert g.metadata[key].type is vt and g.metadata_value(key) == value, key
    assert g.metadata_value("nested") == [[1, -2], []]


def test_quantized_tensors_sizes_alignment_and_mmap(tmp_path):
    rng = np.random.default_rng(5)
    q4 = rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8).tobytes()  # Q4_K 3 rows x 512
    f32 = np.arange(10, dtype=np.float32).tobytes()
    q6 = rng.integers(0, 256, 2 * 210, dtype=np.uint8).tobytes()  # Q6_K, 3-d: 256 x 1 x 2
    p = tmp_path / "q.gguf"
    offs = write_gguf(p, [], [("blk.0.ffn_down.weight", (512, 3), T.Q4_K, q4), ("norm", (10,), T.F32, f32),
                              ("w3", (256, 1, 2), T.Q6_K, q6)], alignment=64)
    g = load_gguf(p, require_supported_tensors=True)
    assert g.alignment == 64 and g.data_start % 64 == 0
    assert [g.tensors[n].absolute_offset for n in ("blk.0.ffn_down.weight", "norm", "w3")] == offs
    assert all(o % 64 == 0 for o in offs)
    t = g.tensors["blk.0.ffn_down.weight"]
    assert t.is_quantized and t.block_size == 256 and t.type_size == 144 and t.nbytes == len(q4)
    assert g.tensors["w3"].nbytes == len(q6) and g.tensors["w3"].numel == 512
    assert [x.name for x in g.quantized_tensors()] == ["blk.0.ffn_down.weight", "w3"]
    for name, payload in (("blk.0.ffn_down.weight", q4), ("norm", f32), ("w3", q6)):
        f, mm, view = g.mmap_tensor(name)
        try:
            assert bytes(view) == payload
        finally:
            view.release()
            mm.close()
            f.close()


def test_partial_last_block_rounds_up(tmp_path):
    p = tmp_path / "r.gguf"
    write_gguf(p, [], [("q8", (40,), T.Q8_0, bytes(2 * 34))])
    assert load_gguf(p).tensors["q8"].nbytes == 2 * 34


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "tensor_type", "value_type", "alignment",
                                  "past_end", "unsized_type"])
def test_malformed_files_fail(tmp_path, case):
    p = tmp_path / "bad.gguf"
    if case == "magic":
        write_gguf(p, [], [], magic=b"GGUG")
    elif case == "version":
        write_gguf(p, [], [], version=4)
    elif case == "truncated":
        write_gguf(p, [("s", V.STRING, "abcdef")], [])
        p.write_bytes(p.read_bytes()[:30])
    elif case == "tensor_type":
        write_gguf(p, [], [("t", (32,), 99, bytes(64))])
    elif case == "value_type":
        write_gguf(p, [], [])
        raw = bytearray(p.read_bytes())
        raw[16:24] = struct.pack("<Q", 1)  # one metadata entry of value type 13
        p.write_bytes(bytes(raw[:24]) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13))
    elif case == "alignment":
        write_gguf(p, [("general.alignment", V.UINT32, 0)], [])
    elif case == "past_end":
        write_gguf(p, [], [("t", (256,), T.Q4_K, bytes(144))])
        p.write_bytes(p.read_bytes()[:-100])
        g = load_gguf(p)
        with pytest.raises(UnsupportedModelError):
            g.mmap_tensor("t")
        return
    else:  # IQ1_M: a known id without a block size
        write_gguf(p, [], [("t", (256,), T.IQ1_M, bytes(56))])
        assert load_gguf(p).tensors["t"].tensor_type is T.IQ1_M
        with pytest.raises(UnsupportedModelError):
            load_gguf(p, require_supported_tensors=True)
        return
    with pytest.raises(UnsupportedModelError):
        load_gguf(p)
