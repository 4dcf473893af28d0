"""Weight files feeding the GPU products through the C ABI: a Stark artifact
written in the converter's layout (tools/converter/stark_convert/compressed.py:143-200)
loaded by stark_qmm_weight_matrix_load (WeightMatrix::load,
crates/stark-engine/src/encodable_block/weight_matrix.rs:114-216) and run by
stark_qmm_encode, and GGUF Q8_0 / Q4_K matrices read by stark_qmm_file_open
(read_gguf, crates/stark-engine/src/engine/hybrid/weights.rs:2770-2865),
uploaded and run by stark_qmm_mapped_many; both against the oracle on the
same bytes."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests import weight_files as WF
from tests.tolerances import check

pytestmark = pytest.mark.gpu


def _mlx(O, rng, n, k, bits, group=64):
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    return O.quantize_affine(w, bits, group, O.GROUP_OUTPUT)


def _run(Q, O, wm, codes, scales, corr, n, k, m, bits, group=64, correction=1, rng=None, label=""):
    x = H.activations(O, rng, m, k)
    st, want = O.matmul(a=x, m=m, n=n, k=k, codes=codes, scales=scales, correction=correction,
                        correction_data=corr, layout=O.GROUP_OUTPUT, row_count=n, group_count=k // group,
                        bits=bits, group_size=group, output_dt=H.F32, threads=8)
    assert st == 0
    d = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    Q.MatmulKernel(H.BF16, H.BF16, H.F32).encode(Q.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=wm.b))
    torch.cuda.synchronize()
    mag = H.dequant_magnitude(O, codes.ravel(), scales.ravel(), corr.ravel() if correction == 1 else corr, n, k, bits,
                              group, 1, correction, H.BF16, x, H.BF16, m)
    check(d.cpu().numpy(), want, mag=mag, label=label)


def test_artifact_fused_qkv_and_down(qmm, oracle, tmp_path):
    """A fused q/k/v matrix (source spans 64 + 32 + 32 rows, W4 g64) and an
    8-bit down matrix, written as model.safetensors with group-output planes
    [G, roundup4(N)], loaded and multiplied at M = 1 and 3."""
    rng = np.random.default_rng(3)
    K = 512
    parts = [_mlx(oracle, rng, r, K, 4) for r in (64, 32, 32)]
    codes = np.concatenate([p[0] for p in parts])
    # fused planes: the converter concatenates rows, then pads to roundup4 (compressed.py:190-197)
    s = np.concatenate([p[1][:, :r] for p, r in zip(parts, (64, 32, 32))], axis=1)
    b = np.concatenate([p[2][:, :r] for p, r in zip(parts, (64, 32, 32))], axis=1)
    dc, ds, db = _mlx(oracle, rng, 200, 256, 8)
    WF.write_artifact(str(tmp_path / "model.safetensors"), {
        "layers.0.attn.qkv.weights": codes, "layers.0.attn.qkv.scales": ("BF16", s),
        "layers.0.attn.qkv.biases": ("BF16", b),
        "layers.0.mlp.down.weights": dc, "layers.0.mlp.down.scales": ("BF16", ds),
        "layers.0.mlp.down.biases": ("BF16", db)})
    f = qmm.WeightFile(str(tmp_path / "model.safetensors"))
    qkv = qmm.WeightMatrix(f, "layers.0.attn.qkv",
                           qmm.WeightMatrixSpec(qmm.SPEC_MLX, 4, 64, source_output_widths=(64, 32, 32)),
                           qmm.OUTPUT_INPUT, 128, K, qmm.BF16)
    assert (qkv.rows, qkv.columns, qkv.source_output_widths) == (128, K, (64, 32, 32))
    down = qmm.WeightMatrix(f, "layers.0.mlp.down", qmm.WeightMatrixSpec(qmm.SPEC_MLX, 8, 64), qmm.OUTPUT_INPUT,
                            200, 256, qmm.BF16)
    for m in (1, 3):
        _run(qmm, oracle, qkv, codes, s, b, 128, K, m, 4, rng=rng, label=f"qkv m{m}")
        _run(qmm, oracle, down, dc, ds, db, 200, 256, m, 8, rng=rng, label=f"down m{m}")
    qkv.free()
    down.free()


def test_artifact_zero_points_and_symmetric(qmm, oracle, tmp_path):
    """IntSpec matrices: zero points (packed U8 plane [G, roundup4(N)/2] for
    4-bit) and symmetric."""
    rng = np.random.default_rng(4)
    n, k, G = 96, 256, 4
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = H.store(oracle, rng.uniform(0.01, 0.1, (G, n)).astype(np.float32).ravel(), H.BF16).reshape(G, n)
    zp = rng.integers(0, 256, (G, n // 2), dtype=np.uint8)
    WF.write_artifact(str(tmp_path / "model.safetensors"), {
        "zp.weights": codes, "zp.scales": ("BF16", s), "zp.zero_points": zp,
        "sym.weights": codes.copy(), "sym.scales": ("BF16", s.copy())})
    f = qmm.WeightFile(str(tmp_path / "model.safetensors"))
    wz = qmm.WeightMatrix(f, "zp", qmm.WeightMatrixSpec(qmm.SPEC_INT, 4, 64), qmm.OUTPUT_INPUT, n, k, qmm.BF16)
    ws = qmm.WeightMatrix(f, "sym", qmm.WeightMatrixSpec(qmm.SPEC_INT, 4, 64, is_symmetric=True), qmm.OUTPUT_INPUT,
                          n, k, qmm.BF16)
    _run(qmm, oracle, wz, codes, s, zp, n, k, 2, 4, correction=2, rng=rng, label="zero points")
    _run(qmm, oracle, ws, codes, s, None, n, k, 2, 4, correction=0, rng=rng, label="symmetric")


def test_artifact_uploads_bytes_unchanged(qmm, oracle, tmp_path):
    """Input-output matrices keep output-group planes [N, G]; the device copy of
    every tensor equals its bytes in the file."""
    rng = np.random.default_rng(5)
    codes, s, b = oracle.quantize_affine(rng.normal(0, 0.02, (64, 128)).astype(np.float32), 4, 64,
                                         oracle.OUTPUT_GROUP)
    WF.write_artifact(str(tmp_path / "model.safetensors"),
                      {"io.weights": codes, "io.scales": ("BF16", s), "io.biases": ("BF16", b)})
    f = qmm.WeightFile(str(tmp_path / "model.safetensors"))
    wm = qmm.WeightMatrix(f, "io", qmm.WeightMatrixSpec(qmm.SPEC_MLX, 4, 64, layout=qmm.INPUT_OUTPUT),
                          qmm.INPUT_OUTPUT, 128, 64, qmm.BF16)
    assert wm.b.raw.params.layout == qmm.OUTPUT_GROUP and (wm.rows, wm.columns) == (64, 128)
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    torch.cuda.synchronize()
    for i, want in enumerate((codes, s, b)):
        host = np.empty(want.nbytes, np.uint8)
        assert hip.hipMemcpy(host.ctypes.data, C.c_void_p(wm._m.device[i]), want.nbytes, 2) == 0  # device to host
        assert np.array_equal(host, np.frombuffer(want.tobytes(), np.uint8))
    wm.free()


@pytest.mark.parametrize("kind", [8, 12])
def test_gguf_file_feeds_mapped_many(qmm, oracle, tmp_path, kind):
    """A GGUF file with a Q8_0 / Q4_K matrix (GGML dims [K, N]) and an F32
    vector; the matrix is uploaded from the mapping and multiplied by
    stark_qmm_mapped_many at M = 1 and 4."""
    rng = np.random.default_rng(kind)
    n, k = 96, 1024
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    blocks = oracle.quantize_q8_0(w) if kind == 8 else oracle.quantize_q4_k(w)
    path = tmp_path / "model.gguf"
    path.write_bytes(WF.gguf_bytes([("blk.0.ffn_up.weight", [k, n], kind, blocks.tobytes()),
                                    ("output_norm.weight", [k], 0, np.ones(k, np.float32).tobytes())],
                                   [("general.architecture", 8, WF.gguf_string("qwen3"))]))
    f = qmm.WeightFile(str(path))
    t = f.tensor("blk.0.ffn_up.weight")
    assert t.shape == (n, k) and t.dtype == kind and t.size == blocks.nbytes
    dev = f.upload("blk.0.ffn_up.weight")
    for m in (1, 4):
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=dev)] * m, inputs=torch.from_numpy(x.ravel()).cuda(),
                                 rows=n, columns=k, format=("packed", kind))
        (out,) = qmm.mapped_many([op])
        got = out.cpu().numpy().reshape(m, n)
        dec = oracle.decode_rows(kind, blocks, n, k)
        for i in range(m):
            check(got[i], oracle.hybrid_packed_matvec(kind, blocks, n, k, x[i]), mag=np.abs(dec) @ np.abs(x[i]),
                  label=f"gguf kind {kind} m{m} row {i}")
    dev.free()
