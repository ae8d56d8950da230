"""A small GGUF v3 writer for tests: metadata + tensors, written from the
published layout (magic, version, counts, key/value table, tensor table,
aligned data section).  Test infrastructure only."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3):
    """metadata: [(key, vtype, value)]; tensors: [(name, ggml_type, ne tuple, bytes)]
    with ne in GGUF order (ne[0] innermost)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vtype, v in metadata:
        out += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offset = 0
    offsets = []
    for name, gtype, ne, data in tensors:
        offsets.append(offset)
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gtype, offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    for (name, gtype, ne, data), off in zip(tensors, offsets):
        assert len(out) % alignment == 0
        out += bytes(data)
        out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(out)
    return bytes(out)


def model_gguf(path, tensors_by_name, n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim,
               extra_meta=(), pattern=None, types=None):
    """Write a gemma-embedding2 GGUF from {name: (array, rows, cols, is_q8)}.
    pattern: the sliding_window_pattern bools (True = sliding; default 5
    sliding + 1 full); types: {name: (ggml type, raw array)} overrides, for
    tensors stored in another type."""
    if pattern is None:
        pattern = [(i + 1) % 6 != 0 for i in range(n_layers)]
    meta = [("general.architecture", STR, "gemma-embedding2"),
            ("gemma-embedding2.block_count", U32, n_layers),
            ("gemma-embedding2.embedding_length", U32, hidden),
            ("gemma-embedding2.feed_forward_length", U32, ffn),
            ("gemma-embedding2.attention.head_count", U32, n_heads),
            ("gemma-embedding2.attention.head_count_kv", ARR, (U32, [n_kv_heads] * n_layers)),
            ("gemma-embedding2.attention.key_length_swa", U32, head_dim),
            ("gemma-embedding2.attention.key_length", U32, head_dim),
            ("gemma-embedding2.attention.layer_norm_rms_epsilon", F32, 1e-6),
            ("gemma-embedding2.rope.freq_base", F32, 1000000.0),
            ("gemma-embedding2.rope.freq_base_swa", F32, 10000.0),
            ("gemma-embedding2.attention.sliding_window_pattern", ARR,
             (BOOL, [bool(p) for p in pattern]))] + list(extra_meta)
    tens = []
    for name, (arr, rows, cols, q8) in tensors_by_name.items():
        gtype = GGML_Q8_0 if q8 else GGML_F32
        if types and name in types:
            gtype, arr = types[name]
        a = np.ascontiguousarray(arr)
        tens.append((name, gtype, (cols, rows) if rows > 1 else (cols,),
                     a.view(np.uint8).tobytes()))
    return write_gguf(path, meta, tens)
