"""The GGUF reader (host code of the library, no GPU): directory, metadata, in-place tensor bytes,
F32 copies, per-block Q8_0 weights under the reference's names and the LM config keys.

Files are written by tests/gguf_writer.py from the published layout.  Pins: the F16 conversion is
checked on every 16-bit pattern against numpy; the Q8_0 conversion against the oracle's dequantizer
(ggml's dequantize_row_q8_0); BF16 by its definition (the top half of an F32).  Malformed files
(bad magic, versions, truncation at every boundary, misaligned or out-of-range tensors, random
corruption) must be refused with a status, never read out of bounds."""
import numpy as np
import pytest

import gguf_writer as W


@pytest.fixture(scope="module")
def vxm():
    import vxm as m

    m.lib()
    return m


def _kv_all():
    return [("general.architecture", W.STR, "voxcpm2"), ("k.u8", W.U8, 200), ("k.i8", W.I8, -100),
            ("k.u16", W.U16, 60000), ("k.i16", W.I16, -30000), ("k.u32", W.U32, 4000000000),
            ("k.i32", W.I32, -123456), ("k.f32", W.F32, 0.125), ("k.bool", W.BOOL, True),
            ("k.u64", W.U64, 7), ("k.i64", W.I64, -9), ("k.f64", W.F64, 2.5),
            ("k.arr", W.ARR, (W.U32, [1, 2, 3])), ("k.arrs", W.ARR, (W.STR, ["a", "bc"])),
            ("k.str", W.STR, "hello")]


def _tensors(orc, rng):
    w = rng.normal(0, 0.02, (3, 64)).astype(np.float32)
    q = orc.quantize_rows(w, orc.QUANT_REF)
    f = rng.normal(0, 1, 40).astype(np.float32)
    h = rng.normal(0, 1, 96).astype(np.float16)
    b = (rng.normal(0, 1, 32).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return [W.q8_tensor("w.q8", q, 3, 64), W.f32_tensor("v.f32", f), ("v.f16", W.GGML_F16, [96], h.tobytes()),
            ("v.bf16", W.GGML_BF16, [32], b.tobytes()), ("t.i32", W.GGML_I32, [5, 2], np.arange(10, dtype=np.int32).tobytes())]


@pytest.mark.parametrize("alignment,version", [(32, 3), (64, 3), (32, 2)])
def test_directory_metadata_and_bytes(vxm, orc, tmp_path, alignment, version):
    rng = np.random.default_rng(alignment + version)
    ts = _tensors(orc, rng)
    p = W.write_gguf(tmp_path / "a.gguf", _kv_all(), ts, alignment=alignment, version=version)
    with vxm.GGUF(p) as g:
        assert g.version == version and len(g) == len(ts)
        for i, (name, gt, ne, raw) in enumerate(ts):
            assert g.find(name) == i
            ti = g.info(name)
            assert ti.name.decode() == name and ti.type == gt and ti.n_dims == len(ne)
            assert list(ti.ne)[:len(ne)] == ne and all(x == 1 for x in list(ti.ne)[len(ne):])
            assert ti.nbytes == len(raw) and ti.offset % alignment == 0 and ti.data % alignment == 0
            assert g.raw(name).tobytes() == raw
        assert g.find("absent") == -1
        assert g.get_i32("k.u8") == 200 and g.get_i32("k.i8") == -100 and g.get_i32("k.u16") == 60000
        assert g.get_i32("k.i16") == -30000 and g.get_i32("k.i32") == -123456 and g.get_i32("k.bool") == 1
        assert g.get_i32("k.u64") == 7 and g.get_i32("k.i64") == -9
        assert g.get_f32("k.f32") == 0.125 and g.get_f32("k.f64") == 2.5 and g.get_f32("k.i32") == -123456.0
        assert g.get_str("k.str") == "hello" and g.get_str("general.architecture") == "voxcpm2"
        assert g.get_i32("missing", 42) == 42 and g.get_f32("missing", 1.5) == 1.5
        assert g.get_str("missing", "dflt") == "dflt" and g.get_str("k.i32", "x") == "x"
        assert g.get_i32("k.str", 5) == 5 and g.get_i32("k.arr", 6) == 6
        if alignment != 32:
            assert g.get_i32("general.alignment") == alignment


def test_f32_copies(vxm, orc, tmp_path):
    rng = np.random.default_rng(3)
    ts = _tensors(orc, rng)
    p = W.write_gguf(tmp_path / "b.gguf", _kv_all(), ts)
    with vxm.GGUF(p) as g:
        assert np.array_equal(g.f32("w.q8"), orc.dequantize_rows(np.frombuffer(ts[0][3], np.uint8), 3, 64).reshape(-1))
        assert np.array_equal(g.f32("v.f32"), np.frombuffer(ts[1][3], np.float32))
        assert np.array_equal(g.f32("v.f16"), np.frombuffer(ts[2][3], np.float16).astype(np.float32))
        bf = np.frombuffer(ts[3][3], np.uint16).astype(np.uint32) << 16
        assert np.array_equal(g.f32("v.bf16").view(np.uint32), bf)
        with pytest.raises(vxm.VxmError):
            g.f32("t.i32")   # integer tensors are not converted


def test_f16_conversion_every_pattern(vxm, tmp_path):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    p = W.write_gguf(tmp_path / "h.gguf", [], [("h", W.GGML_F16, [65536], h.tobytes())])
    with vxm.GGUF(p) as g:
        got = g.f32("h")
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN payloads keep their sign and top mantissa bits
    assert np.array_equal(got[nan].view(np.uint32) >> 13, ref[nan].view(np.uint32) >> 13)


def test_layer_weights_point_into_the_file(vxm, orc, tmp_path):
    from test_gpu_minicpm4 import rand_layer

    rng = np.random.default_rng(5)
    H, nh, nkv, hd, F = 64, 2, 1, 32, 128
    d = rand_layer(orc, rng, H, nh, nkv, hd, F)
    ts = W.voxcpm_block_tensors("base_lm.blk", 3, d, H, nh, nkv, hd, F, norm_type=W.GGML_Q8_0, orc=orc)
    p = W.write_gguf(tmp_path / "l.gguf", [("general.architecture", W.STR, "voxcpm2")], ts)
    cfg = dict(hidden_size=H, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate_size=F)
    with vxm.GGUF(p) as g:
        lw = g.layer_q8_0("base_lm.blk", 3, cfg)
        for key, name in (("q_proj", "self_attn.q_proj.weight"), ("down_proj", "mlp.down_proj.weight")):
            ti = g.info(f"base_lm.blk.3.{name}")
            assert getattr(lw, key) == ti.data
        import ctypes as C

        gin = np.ctypeslib.as_array((C.c_float * H).from_address(lw.input_layernorm))
        gq = orc.dequantize_rows(orc.quantize_rows(d["input_layernorm"][None], orc.QUANT_REF), 1, H)[0]
        assert np.array_equal(gin, gq)
        with pytest.raises(vxm.VxmError) as e:
            g.layer_q8_0("base_lm.blk", 4, cfg)
        assert "base_lm.blk.4.self_attn.q_proj.weight" in str(e.value) and e.value.code == 3
        with pytest.raises(vxm.VxmError):
            g.layer_q8_0("base_lm.blk", 3, dict(cfg, hidden_size=H + 32))   # norm length mismatch


def test_non_q8_projection_is_refused(vxm, orc, tmp_path):
    from test_gpu_minicpm4 import rand_layer

    rng = np.random.default_rng(6)
    d = rand_layer(orc, rng, 64, 2, 1, 32, 128)
    ts = W.voxcpm_block_tensors("residual_lm.blk", 0, d, 64, 2, 1, 32, 128)
    ts[0] = ("residual_lm.blk.0.self_attn.q_proj.weight", W.GGML_F16, [64, 64], np.zeros(64 * 64, np.float16).tobytes())
    p = W.write_gguf(tmp_path / "n.gguf", [], ts)
    with vxm.GGUF(p) as g:
        with pytest.raises(vxm.VxmError) as e:
            g.layer_q8_0("residual_lm.blk", 0, dict(hidden_size=64, n_heads=2, n_kv_heads=1, head_dim=32,
                                                    intermediate_size=128))
        assert e.value.code == 7


@pytest.mark.parametrize("which,ne", [
    (0, [64, 32]),      # q_proj with half its rows
    (3, [32, 64]),      # o_proj with a K that is not n_heads * head_dim
    (6, [64, 64]),      # down_proj whose K is not the FFN width
    (4, [64, 256]),     # gate_proj with more rows than the FFN
])
def test_wrong_shaped_projection_is_refused(vxm, orc, tmp_path, which, ne):
    """A projection whose ne differs from the config's shape is refused with
    VXM_ERR_MODEL_FORMAT before any byte of it is read as weights."""
    from test_gpu_minicpm4 import rand_layer

    rng = np.random.default_rng(7 + which)
    H, nh, nkv, hd, F = 64, 2, 1, 32, 128
    d = rand_layer(orc, rng, H, nh, nkv, hd, F)
    ts = W.voxcpm_block_tensors("base_lm.blk", 0, d, H, nh, nkv, hd, F)
    name = ts[which][0]
    q = orc.quantize_rows(rng.normal(0, 0.02, (ne[1], ne[0])).astype(np.float32), orc.QUANT_REF)
    ts[which] = W.q8_tensor(name, q, ne[1], ne[0])
    p = W.write_gguf(tmp_path / "s.gguf", [("general.architecture", W.STR, "voxcpm2")], ts)
    cfg = dict(hidden_size=H, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate_size=F)
    with vxm.GGUF(p) as g:
        with pytest.raises(vxm.VxmError) as e:
            g.layer_q8_0("base_lm.blk", 0, cfg)
        assert e.value.code == 3 and name in str(e.value), str(e.value)


def test_missing_intermediate_size_key_is_caught_by_the_shape_check(vxm, orc, tmp_path):
    """Without voxcpm.intermediate_size the config takes the reference's
    default (8192); a file whose real FFN is narrower is then refused at the
    layer load instead of being read past its gate / up / down tensors."""
    from test_gpu_minicpm4 import rand_layer

    rng = np.random.default_rng(8)
    H, nh, nkv, hd, F = 64, 2, 1, 32, 128
    d = rand_layer(orc, rng, H, nh, nkv, hd, F)
    ts = W.voxcpm_block_tensors("base_lm.blk", 0, d, H, nh, nkv, hd, F)
    kv = [("general.architecture", W.STR, "voxcpm2"), ("voxcpm.hidden_size", W.I32, H),
          ("voxcpm.num_attention_heads", W.I32, nh), ("voxcpm.num_kv_heads", W.I32, nkv),
          ("voxcpm.head_dim", W.I32, hd)]
    p = W.write_gguf(tmp_path / "k.gguf", kv, ts)
    with vxm.GGUF(p) as g:
        cfg = g.minicpm4_config()
        assert cfg["intermediate_size"] == 8192
        with pytest.raises(vxm.VxmError) as e:
            g.layer_q8_0("base_lm.blk", 0, cfg)
        assert e.value.code == 3 and "mlp.gate_proj" in str(e.value), str(e.value)


def test_minicpm4_config_defaults_and_sanitisation(vxm, tmp_path):
    p = W.write_gguf(tmp_path / "c0.gguf", [("general.architecture", W.STR, "voxcpm2")], [])
    with vxm.GGUF(p) as g:
        c = g.minicpm4_config()
        assert (c["hidden_size"], c["n_layers"], c["n_heads"], c["n_kv_heads"], c["intermediate_size"],
                c["head_dim"], c["rope_theta"], c["no_rope"]) == (2048, 24, 16, 4, 8192, 128, 1000000, 0)
        assert c["rms_norm_eps"] == np.float32(1e-6) and c["scale_depth"] == 0
        r = g.minicpm4_config(residual=True)
        assert (r["hidden_size"], r["n_layers"], r["n_heads"], r["n_kv_heads"], r["no_rope"], r["rope_theta"]) == \
            (2048, 8, 16, 4, 1, 0)
    kv = [("general.architecture", W.STR, "voxcpm2"), ("voxcpm.hidden_size", W.I32, 1024),
          ("voxcpm.num_hidden_layers", W.I32, 28), ("voxcpm.num_kv_heads", W.I32, 2),
          ("voxcpm.intermediate_size", W.I32, 6144), ("voxcpm.rms_norm_eps", W.F32, 0.0),
          ("voxcpm.rope_theta", W.I32, 10000), ("voxcpm.scale_depth", W.F32, 1.4),
          ("voxcpm.res_num_layers", W.I32, 6), ("voxcpm.res_scale_depth", W.F32, 1.4)]
    for mup in (False, True):
        p = W.write_gguf(tmp_path / f"c{int(mup)}.gguf", kv + [("voxcpm.use_mup", W.BOOL, mup)], [])
        with vxm.GGUF(p) as g:
            c = g.minicpm4_config()
            assert (c["hidden_size"], c["n_layers"], c["n_kv_heads"], c["intermediate_size"], c["rope_theta"]) == \
                (1024, 28, 2, 6144, 10000)
            assert c["rms_norm_eps"] == np.float32(1e-5)          # 0 in the file -> 1e-5
            assert c["scale_depth"] == (np.float32(1.4) if mup else 0.0)
            r = g.minicpm4_config(residual=True)
            assert r["n_layers"] == 6 and r["scale_depth"] == (np.float32(1.4) if mup else 0.0)
    p = W.write_gguf(tmp_path / "x.gguf", [("general.architecture", W.STR, "llama")], [])
    with vxm.GGUF(p) as g:
        with pytest.raises(vxm.VxmError) as e:
            g.minicpm4_config()
        assert e.value.code == 4


def _open_code(vxm, path):
    try:
        vxm.GGUF(path).close()
        return 0
    except vxm.VxmError as e:
        return e.code


def test_malformed_files_are_refused(vxm, orc, tmp_path):
    rng = np.random.default_rng(7)
    good = W.gguf_bytes(_kv_all(), _tensors(orc, rng))
    p = tmp_path / "m.gguf"
    assert _open_code(vxm, tmp_path / "does_not_exist.gguf") == 2
    p.write_bytes(b"GGUX" + good[4:])
    assert _open_code(vxm, p) == 3
    for v in (1, 4):
        p.write_bytes(good[:4] + np.uint32(v).tobytes() + good[8:])
        assert _open_code(vxm, p) == 3
    # every truncation short of the last tensor's end is refused
    last_end = len(good) - ((-len(np.arange(10, dtype=np.int32).tobytes())) % 32)
    for cut in list(range(0, 600, 7)) + list(range(last_end - 40, last_end)):
        p.write_bytes(good[:cut])
        assert _open_code(vxm, p) in (2, 3), cut
    # a tensor whose data lies past the end, a misaligned offset, a huge count
    bad = W.gguf_bytes([], [("a", W.GGML_F32, [1 << 20], b"\0" * 16)])
    p.write_bytes(bad[:len(bad) - (len(bad) % 32)] + b"\0" * 64)
    assert _open_code(vxm, p) == 3
    body = W.gguf_bytes([], [("a", W.GGML_F32, [4], b"\0" * 16)])
    i = body.index(b"a") + 1 + 4 + 8 + 4   # name, n_dims, ne[0], type -> offset field
    p.write_bytes(body[:i] + np.uint64(4).tobytes() + body[i + 8:])
    assert _open_code(vxm, p) == 3
    p.write_bytes(good[:8] + np.uint64(1 << 40).tobytes() + good[16:])
    assert _open_code(vxm, p) == 3


def test_random_corruption_never_reads_out_of_bounds(vxm, orc, tmp_path):
    """Corrupt bytes of the header and directory: every open returns a status (0 or an error); a read
    out of the mapping would fault this process."""
    rng = np.random.default_rng(8)
    good = bytearray(W.gguf_bytes(_kv_all(), _tensors(orc, rng)))
    p = tmp_path / "r.gguf"
    head = len(good) - 400
    for _ in range(300):
        b = bytearray(good)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        p.write_bytes(bytes(b))
        assert _open_code(vxm, p) in (0, 3)
