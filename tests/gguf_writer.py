"""A minimal GGUF (v2 / v3) writer for test fixtures, written from ggml's published file layout:
"GGUF", u32 version, u64 tensor count, u64 key/value count, the key/value pairs (u64-length string
key, u32 value type, value), the tensor infos (name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
u64 offset into the data section), zero padding to the alignment, then the tensor data, each
tensor at an aligned offset.  Little-endian throughout."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}

GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16, GGML_I32 = 0, 1, 8, 30, 26


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kv, tensors, alignment=32, version=3, set_alignment_key=None):
    """kv: list of (key, type, value); tensors: list of (name, ggml_type, ne list, raw bytes).
    Returns the file contents."""
    kv = list(kv)
    add_key = (alignment != 32) if set_alignment_key is None else set_alignment_key
    if add_key:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv)
    offs, off = [], 0
    for _, _, _, raw in tensors:
        offs.append(off)
        off = (off + len(raw) + alignment - 1) // alignment * alignment
    for (name, gt, ne, raw), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", e) for e in ne)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    data = bytearray(off)
    for (_, _, _, raw), o in zip(tensors, offs):
        data[o:o + len(raw)] = raw
    return head + b"\0" * pad + bytes(data)


def write_gguf(path, kv, tensors, **kw):
    with open(path, "wb") as f:
        f.write(gguf_bytes(kv, tensors, **kw))
    return path


def q8_tensor(name, q8_rows, n_rows, k):
    """A 2-D Q8_0 tensor from GGUF row bytes: ne = [k, n_rows]."""
    return (name, GGML_Q8_0, [k, n_rows], np.ascontiguousarray(q8_rows, np.uint8).tobytes())


def f32_tensor(name, a):
    a = np.ascontiguousarray(a, np.float32)
    return (name, GGML_F32, list(a.shape[::-1]), a.tobytes())


def voxcpm_block_tensors(prefix, layer, d, H, nh, nkv, hd, F, norm_type=GGML_F32, orc=None):
    """The nine tensors of one block as the reference names them; d holds GGUF Q8_0 rows and F32 gains
    (as rand_layer builds them).  norm_type Q8_0 stores the gains quantized, as the reference's quantize
    tool does for every 1-D tensor whose length is a multiple of 32."""
    out = []
    names = [("q_proj", "self_attn.q_proj.weight", nh * hd, H), ("k_proj", "self_attn.k_proj.weight", nkv * hd, H),
             ("v_proj", "self_attn.v_proj.weight", nkv * hd, H), ("o_proj", "self_attn.o_proj.weight", H, nh * hd),
             ("gate_proj", "mlp.gate_proj.weight", F, H), ("up_proj", "mlp.up_proj.weight", F, H),
             ("down_proj", "mlp.down_proj.weight", H, F)]
    for key, suffix, n_rows, k in names:
        raw = np.ascontiguousarray(d[key], np.uint8)
        assert raw.size == n_rows * k // 32 * 34
        out.append(q8_tensor(f"{prefix}.{layer}.{suffix}", raw, n_rows, k))
    for key, suffix in (("input_layernorm", "input_layernorm.weight"),
                        ("post_attention_layernorm", "post_attention_layernorm.weight")):
        g = np.ascontiguousarray(d[key], np.float32)
        if norm_type == GGML_Q8_0:
            out.append((f"{prefix}.{layer}.{suffix}", GGML_Q8_0, [g.size],
                        orc.quantize_rows(g[None], orc.QUANT_REF).tobytes()))
        else:
            out.append(f32_tensor(f"{prefix}.{layer}.{suffix}", g))
    return out
