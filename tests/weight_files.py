"""Writers of small weight files for the loader tests: GGUF v3 (the layout the
reference's own fixtures write, crates/stark-engine/src/engine/hybrid/weights.rs:4299-4338)
and Stark's converted safetensors artifact (tools/converter/stark_convert/compressed.py:143-200:
`<prefix>.weights` U8 [N, K*bits/8], `.scales` / `.biases` [G, roundup4(N)] for
output-input matrices, [N, G] for input-output ones)."""
import struct

import numpy as np


def gguf_string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def gguf_bytes(tensors, metadata=(), alignment=32, truncate=0, version=3, offsets=None):
    """tensors: [(name, ggml dims innermost first, kind, payload bytes)];
    metadata: [(key, gguf type, packed value bytes)]; offsets overrides the
    recorded data offsets (the payload is still laid out back to back)."""
    out = b"GGUF" + struct.pack("<I", version) + struct.pack("<QQ", len(tensors), len(metadata))
    for key, kind, value in metadata:
        out += gguf_string(key) + struct.pack("<I", kind) + value
    offset = 0
    infos, payload = b"", b""
    for i, (name, dims, kind, data) in enumerate(tensors):
        infos += gguf_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", kind, offset if offsets is None else offsets[i])
        pad = (-len(data)) % alignment if i + 1 < len(tensors) else 0  # no padding after the last payload
        payload += data + b"\0" * pad
        offset += len(data) + pad
    out += infos
    out += b"\0" * ((-len(out)) % alignment)
    out += payload
    return out[:len(out) - truncate] if truncate else out


def u64(v):
    return struct.pack("<Q", v)


def u16(v):
    return struct.pack("<H", v)


def write_artifact(path, tensors, metadata=None):
    """tensors: {name: numpy array (uint8, or uint16 holding bf16 bits with
    dtype tag 'BF16', or float16/float32)}; written with the safetensors
    package's numpy writer, bf16 planes via torch."""
    import torch
    from safetensors.torch import save_file
    out = {}
    for name, a in tensors.items():
        if isinstance(a, tuple):  # ("BF16", uint16 bits)
            out[name] = torch.from_numpy(np.ascontiguousarray(a[1]).view(np.int16)).view(torch.bfloat16)
        else:
            out[name] = torch.from_numpy(np.ascontiguousarray(a))
    save_file(out, path, metadata=metadata)
