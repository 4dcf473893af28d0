"""Weight files through the C ABI, on the CPU (parsing and validation need no
device): GGUF v3 headers as the hybrid engine reads them
(crates/stark-engine/src/engine/hybrid/weights.rs:815-895, 2686-2865), Stark
artifacts as ParameterLoader indexes them (crates/stark-engine/src/parameters/loader.rs:80-127,
safetensors_metadata.rs:113-128), and WeightMatrix::load's argument checks
(crates/stark-engine/src/encodable_block/weight_matrix.rs:53-216), which all
fail before any device copy."""
import os
import struct

import numpy as np
import pytest

from tests import weight_files as WF


@pytest.fixture(scope="module")
def Q():
    from stark_amd import qmm
    qmm.lib()
    return qmm


def _reference_gguf(splits=1, truncate=False):
    """The reference's own fixture (weights.rs:4299-4338): split metadata and one
    Q8_0 'matrix' of GGML dims [32, 2], block scales 1.0 and 0.5 over codes 0..31."""
    meta = [("split.no", 2, WF.u16(0)), ("split.count", 2, WF.u16(splits))]
    data = b"".join(WF.u16(s) + bytes(range(32)) for s in (0x3C00, 0x3800))
    return WF.gguf_bytes([("matrix", [32, 2], 8, data)], meta, truncate=1 if truncate else 0)


def test_gguf_reference_fixture_rows(Q, oracle, tmp_path):
    """weights.rs:4341-4355: shape [2, 32], rows 0..31 and 0.5 * (0..31); a
    split count of 2 with one file and a truncated payload are rejected."""
    p = tmp_path / "model.gguf"
    p.write_bytes(_reference_gguf())
    f = Q.WeightFile(str(p))
    assert f.kind == Q.WeightFile.GGUF and f.names() == ["matrix"]
    t = f.tensor("matrix")
    assert t.dtype == 8 and t.shape == (2, 32) and t.size == 68 and t.offset % 32 == 0
    rows = oracle.decode_rows(8, np.frombuffer(f.host_bytes("matrix"), np.uint8), 2, 32)
    assert np.array_equal(rows[0], np.arange(32, dtype=np.float32))
    assert np.array_equal(rows[1], 0.5 * np.arange(32, dtype=np.float32))
    assert f.metadata("split.count") == "1"
    f.close()
    p.write_bytes(_reference_gguf(splits=2))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(p))
    assert "incomplete GGUF split set" in e.value.detail
    p.write_bytes(_reference_gguf(truncate=True))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(p))
    assert e.value.detail == "truncated GGUF tensor"


@pytest.mark.parametrize("kind", [101, 102, 103, 104])
def test_gguf_rejects_private_integer_tags(Q, tmp_path, kind):
    """weights.rs:4357-4386: the safetensors-only integer tags are never GGML kinds."""
    p = tmp_path / "model.gguf"
    p.write_bytes(WF.gguf_bytes([("t", [1], kind, b"\0" * (8 if kind == 102 else 4))]))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(p))
    assert e.value.status == Q.UNSUPPORTED and e.value.detail == "unsupported GGUF tensor type"


def test_gguf_header_checks(Q, tmp_path):
    p = tmp_path / "model.gguf"
    blk = WF.u16(0x3C00) + bytes(32)
    cases = [
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], version=2), "GGUF version three is required"),
        (b"GGUX" + WF.gguf_bytes([("m", [32, 1], 8, blk)])[4:], "GGUF version three is required"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk), ("m", [32, 1], 8, blk)]), "duplicate GGUF tensor"),
        (WF.gguf_bytes([("m", [31, 1], 8, blk)]), "weight dimension is not block aligned"),
        (WF.gguf_bytes([("m", [32, 0], 8, blk)]), "empty tensor dimension"),
        (WF.gguf_bytes([("", [32, 1], 8, blk)]), "invalid GGUF tensor identity or rank"),
        (WF.gguf_bytes([("m", [32, 1, 1, 1, 1], 8, blk)]), "invalid GGUF tensor identity or rank"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("general.alignment", 4, struct.pack("<I", 48))]),
         "invalid GGUF alignment"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("k", 7, b"\x02")]), "invalid GGUF boolean"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("k", 6, struct.pack("<f", float("inf")))]),
         "nonfinite GGUF metadata"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("k", 9, struct.pack("<IQ", 9, 0))]), "nested GGUF arrays"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("k", 13, b"")]), "unsupported GGUF metadata type"),
        (WF.gguf_bytes([("m", [32, 1], 8, blk)], [("k", 8, WF.gguf_string("a")), ("k", 8, WF.gguf_string("b"))]),
         "duplicate GGUF metadata"),
    ]
    for data, msg in cases:
        p.write_bytes(data)
        with pytest.raises(Q.WeightFileError) as e:
            Q.WeightFile(str(p))
        assert e.value.detail == msg, (msg, e.value.detail)
    # overlapping payloads: the second tensor recorded at the first one's offset
    p.write_bytes(WF.gguf_bytes([("a", [32, 1], 8, blk), ("b", [32, 1], 8, blk)], offsets=[0, 0]))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(p))
    assert e.value.detail == "overlapping GGUF tensors"
    p.write_bytes(WF.gguf_bytes([("a", [32, 1], 8, blk)], offsets=[16]))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(p))
    assert e.value.detail == "unaligned GGUF tensor"


def test_gguf_metadata_and_alignment(Q, tmp_path):
    blk = WF.u16(0x3C00) + bytes(32)
    meta = [("general.alignment", 4, struct.pack("<I", 64)), ("general.name", 8, WF.gguf_string("tiny")),
            ("tokens", 9, struct.pack("<IQ", 4, 3) + struct.pack("<III", 7, 8, 9)),
            ("rope", 6, struct.pack("<f", 0.5)), ("flag", 7, b"\x01")]
    p = tmp_path / "model.gguf"
    p.write_bytes(WF.gguf_bytes([("w", [32, 3], 8, blk * 3), ("v", [4], 0, bytes(16))], meta, alignment=64))
    f = Q.WeightFile(str(p))
    assert f.metadata("general.name") == "tiny" and f.metadata("tokens") == "[7,8,9]"
    assert f.metadata("rope") == "0.5" and f.metadata("flag") == "true"
    assert f.tensor("w").offset % 64 == 0 and f.tensor("v").offset % 64 == 0
    assert f.tensor("v").dtype == 0 and f.tensor("v").shape == (4,)
    with pytest.raises(Q.WeightFileError) as e:
        f.metadata("missing")
    assert e.value.status == Q.KEY_NOT_FOUND


def test_gguf_split_directory(Q, tmp_path):
    """A directory of split files: split.no / split.count complete, metadata
    from split 0, tensors from every split; '._' files are skipped."""
    blk = WF.u16(0x3C00) + bytes(32)

    def split(no, count, name):
        return WF.gguf_bytes([(name, [32, 1], 8, blk)], [("split.no", 2, WF.u16(no)), ("split.count", 2, WF.u16(count)),
                                                          ("split.tensors.count", 4, struct.pack("<I", count))])
    (tmp_path / "m-00001.gguf").write_bytes(split(0, 2, "a"))
    (tmp_path / "m-00002.gguf").write_bytes(split(1, 2, "b"))
    (tmp_path / "._m-00001.gguf").write_bytes(b"AppleDouble metadata")
    f = Q.WeightFile(str(tmp_path))
    assert f.names() == ["a", "b"] and f.metadata("split.no") == "0"
    f.close()
    (tmp_path / "m-00002.gguf").write_bytes(split(0, 2, "b"))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(tmp_path))
    assert e.value.detail == "invalid or duplicate GGUF split"


# ----------------------------------------------------------------- safetensors artifact

def _artifact(tmp_path, **extra):
    rng = np.random.default_rng(0)
    t = {"layer.weights": rng.integers(0, 256, (48, 64), dtype=np.uint8),
         "layer.scales": ("BF16", rng.integers(0, 1 << 15, (2, 48), dtype=np.uint16)),
         "layer.biases": ("BF16", rng.integers(0, 1 << 15, (2, 48), dtype=np.uint16))}
    t.update(extra)
    p = str(tmp_path / "model.safetensors")
    WF.write_artifact(p, t, metadata={"format": "stark"})
    return p, t


def test_artifact_index(Q, tmp_path):
    p, t = _artifact(tmp_path)
    f = Q.WeightFile(p)
    assert f.kind == Q.WeightFile.SAFETENSORS and f.names() == sorted(t)
    info = f.tensor("layer.weights")
    assert info.dtype == Q.U8 and info.shape == (48, 64) and info.size == 48 * 64
    assert f.host_bytes("layer.weights") == t["layer.weights"].tobytes()
    s = f.tensor("layer.scales")
    assert s.dtype == Q.BF16 and s.shape == (2, 48)
    assert f.host_bytes("layer.scales") == t["layer.scales"][1].tobytes()
    assert f.metadata("format") == "stark"


def test_artifact_header_errors(Q, tmp_path):
    p, _ = _artifact(tmp_path)
    data = open(p, "rb").read()
    q = tmp_path / "bad.safetensors"
    q.write_bytes(data[:-1])  # payload past the end of the file
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(q))
    assert e.value.status == Q.HEADER_ERROR and e.value.detail == "Tensor payload exceeds file length"
    q.write_bytes(struct.pack("<Q", 100000001) + data[8:])
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(q))
    assert e.value.detail == "The header is too large."
    q.write_bytes(struct.pack("<Q", 7) + b'{"a":1}')
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(q))
    assert e.value.status == Q.HEADER_ERROR
    hdr = b'{"x":{"dtype":"F64","shape":[1],"data_offsets":[0,8]}}'
    q.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(8))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(q))
    assert e.value.detail == "Unsupported safetensors dtype: F64"
    hdr = b'{"x":{"dtype":"F32","shape":[1],"data_offsets":[8,4]}}'
    q.write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(8))
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightFile(str(q))
    assert e.value.detail.startswith("Invalid data offsets for tensor x")


def _load(Q, f, spec, out_dim=48, in_dim=128, layout=None, dt=None):
    return Q.WeightMatrix(f, "layer", spec, spec.layout if layout is None else layout, out_dim, in_dim,
                          Q.BF16 if dt is None else dt)


def test_weight_matrix_load_validation(Q, tmp_path):
    """WeightMatrix::load's checks, in its order, each before any device copy."""
    p, _ = _artifact(tmp_path)
    f = Q.WeightFile(p)
    S = Q.WeightMatrixSpec
    cases = [
        (S(Q.SPEC_MLX, bits=3), {}, Q.UNSUPPORTED_CONFIGURATION),                 # parse_spec: bits
        (S(Q.SPEC_MLX, group_size=0), {}, Q.UNSUPPORTED_CONFIGURATION),           # zero group
        (S(Q.SPEC_MLX, bits=5, group_size=32), {}, Q.UNSUPPORTED_CONFIGURATION),  # U5 needs group 64
        (S(Q.SPEC_INT, bits=5), {}, Q.UNSUPPORTED_CONFIGURATION),                 # U5 only with biases
        (S(Q.SPEC_MLX, materialize_affine_input_sum=True, bits=8), {}, Q.UNSUPPORTED_CONFIGURATION),
        (S(Q.SPEC_MLX), dict(layout=Q.INPUT_OUTPUT), Q.UNSUPPORTED_CONFIGURATION),  # required layout
        (S(Q.SPEC_MLX, source_output_widths=(16, 16)), {}, Q.UNSUPPORTED_CONFIGURATION),  # spans != rows
        (S(Q.SPEC_MLX, source_output_widths=(16, 0, 32)), {}, Q.UNSUPPORTED_CONFIGURATION),
        (S(Q.SPEC_MLX), dict(out_dim=47), Q.INVALID_TENSOR),                       # weights shape
        (S(Q.SPEC_MLX, bits=8), {}, Q.INVALID_TENSOR),                             # row bytes for 8 bits
        (S(Q.SPEC_MLX), dict(dt=Q.F16), Q.INVALID_TENSOR),                         # plane dtype
        (S(Q.SPEC_INT, is_symmetric=False), {}, Q.KEY_NOT_FOUND),                  # no zero_points tensor
        (S(Q.SPEC_MLX, layout=Q.INPUT_OUTPUT), dict(out_dim=128, in_dim=48), Q.INVALID_TENSOR),  # [N, G] planes
    ]
    for spec, kw, status in cases:
        with pytest.raises(Q.WeightFileError) as e:
            _load(Q, f, spec, **kw)
        assert e.value.status == status, (spec, kw, e.value.detail)
    with pytest.raises(Q.WeightFileError) as e:
        Q.WeightMatrix(f, "missing", S(Q.SPEC_MLX), Q.OUTPUT_INPUT, 48, 128, Q.BF16)
    assert e.value.status == Q.KEY_NOT_FOUND and e.value.detail == 'Array with key "missing.weights" not found.'
