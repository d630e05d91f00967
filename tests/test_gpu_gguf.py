"""A MiniCPM4 stack loaded from a GGUF file (weights used in place from the mapping, norms stored as
Q8_0 the way the reference's quantize tool writes every 1-D tensor) runs bit-identically to the same
stack built from the arrays, with the gains the reference's loader would dequantize
(vcpm_model_ensure_f32, src/model_loader.c:254-352).  The small shape takes the per-op kernels, the
decode shape the single-launch kernel."""
import numpy as np
import pytest

import gguf_writer as W
from test_gpu_minicpm4 import _dev, rand_layer

pytestmark = pytest.mark.gpu


def _dq(orc, g):
    return orc.dequantize_rows(orc.quantize_rows(np.asarray(g, np.float32)[None], orc.QUANT_REF), 1, g.size)[0]


@pytest.mark.parametrize("H,nh,nkv,hd,F", [(256, 4, 2, 64, 512), (2048, 16, 2, 128, 6144)])
def test_stack_from_gguf_matches_arrays(vxm_ctx, orc, tmp_path, H, nh, nkv, hd, F):
    import vxm

    L = 2
    rng = np.random.default_rng(H + F)
    layers = [rand_layer(orc, rng, H, nh, nkv, hd, F) for _ in range(L)]
    fnorm = (1 + rng.normal(0, 0.02, H)).astype(np.float32)
    ts = []
    for l, d in enumerate(layers):
        ts += W.voxcpm_block_tensors("base_lm.blk", l, d, H, nh, nkv, hd, F, norm_type=W.GGML_Q8_0, orc=orc)
    ts.append(("base_lm.norm.weight", W.GGML_Q8_0, [H], orc.quantize_rows(fnorm[None], orc.QUANT_REF).tobytes()))
    kv = [("general.architecture", W.STR, "voxcpm2"), ("voxcpm.hidden_size", W.I32, H),
          ("voxcpm.num_hidden_layers", W.I32, L), ("voxcpm.num_attention_heads", W.I32, nh),
          ("voxcpm.num_kv_heads", W.I32, nkv), ("voxcpm.intermediate_size", W.I32, F),
          ("voxcpm.head_dim", W.I32, hd), ("voxcpm.rope_theta", W.I32, 10000),
          ("voxcpm.rms_norm_eps", W.F32, 1e-6)]
    path = W.write_gguf(tmp_path / "m.gguf", kv, ts)
    with vxm.GGUF(path) as g:
        cfg = g.minicpm4_config()
        assert (cfg["hidden_size"], cfg["n_layers"], cfg["n_heads"], cfg["intermediate_size"]) == (H, L, nh, F)
        a = vxm.MiniCPM4(vxm_ctx, cfg, [g.layer_q8_0("base_lm.blk", l, cfg) for l in range(L)],
                         final_norm=g.f32("base_lm.norm.weight"))
    arr = [dict(d, input_layernorm=_dq(orc, d["input_layernorm"]),
                post_attention_layernorm=_dq(orc, d["post_attention_layernorm"])) for d in layers]
    b = vxm.MiniCPM4(vxm_ctx, cfg, arr, final_norm=_dq(orc, fnorm))
    cap = 64
    kva, kvb = vxm.KVCache(vxm_ctx, L, nkv, hd, cap), vxm.KVCache(vxm_ctx, L, nkv, hd, cap)
    x0 = rng.normal(0, 1, (5, H)).astype(np.float32)
    xa, xb = _dev(x0), _dev(x0)
    a.forward(kva, xa, 0)
    b.forward(kvb, xb, 0)
    assert np.array_equal(xa.cpu().numpy(), xb.cpu().numpy())
    for pos in range(5, 8):
        t = rng.normal(0, 1, (1, H)).astype(np.float32)
        ya, yb = _dev(t), _dev(t)
        a.forward(kva, ya, pos)
        b.forward(kvb, yb, pos)
        a.check()
        assert np.array_equal(ya.cpu().numpy(), yb.cpu().numpy()), pos
    for o in (a, b, kva, kvb):
        o.free()
