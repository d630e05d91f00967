"""GPU parity at the measured workloads' full sizes, against the oracle.

The MiniCPM4 TSLM shape (hidden 2048, 16 q / 2 kv heads of 128, SwiGLU 6144,
Q8_0 weights ~ N(0, 0.02)) at full depth (28 layers):
  * the 28-layer decode of consecutive tokens from context 256 on the
    single-launch (persistent) kernel and on the one-kernel-per-op path
    (vcpm_minicpm4_forward with n_tokens = 1, src/minicpm4.c:536-572), with
    the appended KV rows of the first, a middle and the last layer;
  * the 512-token prompt prefill (the M = n_tokens GEMMs of
    gen_prompt_eval_range, src/gen_prompt.c:186-272): per layer, each device
    block fed the oracle its own input; the whole 28-layer stack against the
    oracle's; and 512 tokens in one call against two chunks of 256.

Bars.  A single block fed identical inputs is held to the prefill block bar
(>= 99% of elements within 1e-3 rel / 1e-4 abs, every element within 4 BF16
ulps, relative L2 <= 1e-3; the MFMA attention sums up to 512 scores and P.V
products in its own order).  A multi-layer stack compounds BF16 rounding
flips (one flipped activation changes every later Q8_0 block it enters), so
stacks are held to the decode-stack bar: cosine >= 0.9995 and relative L2
<= 2e-2, beside the oracle's own sensitivity to a one-ulp input change,
which is printed for scale.
"""
import numpy as np
import pytest

from test_gpu_decode import assert_stack_close
from test_gpu_minicpm4 import _dev, assert_layer_close, cfg_dict, orc_cfg, to_orc

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, F, L = 2048, 16, 2, 128, 6144, 28


def make_layers(vxm, seed, n_layers):
    """Seeded Q8_0 layers (GGUF rows) and gains from the library's host generator
    (SplitMix64 + Box-Muller, the _ref weight rule)."""
    qd, kvd = NH * HD, NKV * HD
    shapes = [("q_proj", qd, H), ("k_proj", kvd, H), ("v_proj", kvd, H), ("o_proj", H, qd),
              ("gate_proj", F, H), ("up_proj", F, H), ("down_proj", H, F)]
    per_layer = sum(n * k for _, n, k in shapes) + 2 * H
    layers = []
    for l in range(n_layers):
        off = l * per_layer
        d = {}
        for name, n, k in shapes:
            d[name] = vxm.host_quantize_q8_0(vxm.host_randn(seed, n * k, 0.0, 0.02, offset=off).reshape(n, k))
            off += n * k
        d["input_layernorm"] = vxm.host_randn(seed, H, 1.0, 0.02, offset=off)
        d["post_attention_layernorm"] = vxm.host_randn(seed, H, 1.0, 0.02, offset=off + H)
        layers.append(d)
    return layers


@pytest.fixture(scope="module")
def stack28():
    import vxm

    layers = make_layers(vxm, 1, L)
    fn = vxm.host_randn(2, H, 1.0, 0.02)
    return layers, fn


def _prior_cache(orc, rng, cap, ctx0):
    k = np.zeros((NKV, cap, HD), np.uint16)
    v = np.zeros_like(k)
    if ctx0:
        k[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (NKV, ctx0, HD)).astype(np.float32)))
        v[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (NKV, ctx0, HD)).astype(np.float32)))
    return k, v


def _kv_rows_close(orc, got_bits, want_bits, rows, what, bar=2e-2):
    g = orc.fp16_bits_to_fp32(got_bits)[:, rows].astype(np.float64)
    w = orc.fp16_bits_to_fp32(want_bits)[:, rows].astype(np.float64)
    rel = np.linalg.norm(g - w) / np.linalg.norm(w)
    eq = float((got_bits[:, rows] == want_bits[:, rows]).mean())
    print(f"{what}: rel-L2 {rel:.3g}, identical {eq:.4f}")
    assert rel <= bar, (what, rel)
    return eq


def _oracle_sensitivity(orc, oc, ol, fn, x, kcs, vcs, cap, pos, ref):
    """How far the oracle's own output moves when one input element moves by one
    BF16 ulp (printed for scale beside the device's deviation)."""
    xp = x.copy()
    xp.flat[7] = np.float32(xp.flat[7] * (1 + 2.0 ** -7))
    kc = [k.copy() for k in kcs]
    vc = [v.copy() for v in vcs]
    alt = orc.minicpm4_forward(oc, ol, fn, xp, kc, vc, cap, pos)
    return float(np.linalg.norm(alt - ref) / np.linalg.norm(ref))


def test_decode_28_layers_4_tokens_from_ctx256(vxm_ctx, orc, stack28):
    """The 28-layer decode workload (context 256 -> 260): the persistent kernel and
    the per-op path each against the oracle, token by token, and the KV rows they
    append at layers 0, 13 and 27."""
    import vxm

    layers, fn = stack28
    cap, ctx0, steps = 512, 256, 4
    rng = np.random.default_rng(303)
    c = cfg_dict(H, L, NH, NKV, HD, F)
    oc = orc_cfg(orc, c)
    ol = [to_orc(orc, d) for d in layers]
    models, kvs = {}, {}
    kcs, vcs = [], []
    for mode in (2, 1):
        models[mode] = vxm.MiniCPM4(vxm_ctx, c, layers, final_norm=fn)
        models[mode].set_decode_mode(mode)
        kvs[mode] = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
    for l in range(L):
        k, v = _prior_cache(orc, rng, cap, ctx0)
        for mode in (2, 1):
            kvs[mode].upload(l, k, v)
        kcs.append(k.reshape(-1).copy())
        vcs.append(v.reshape(-1).copy())
    try:
        for t in range(steps):
            x = rng.normal(0, 1, (1, H)).astype(np.float32)
            outs = {}
            for mode in (2, 1):
                xd = _dev(x)
                models[mode].forward(kvs[mode], xd, ctx0 + t)
                vxm_ctx.sync()
                outs[mode] = xd.cpu().numpy()
            models[2].check()
            if t == 0:
                kc0 = [k.copy() for k in kcs]
                vc0 = [v.copy() for v in vcs]
            ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0 + t)
            if t == 0:
                sens = _oracle_sensitivity(orc, oc, ol, fn, x, kc0, vc0, cap, ctx0, ref)
                print(f"oracle: one BF16 ulp on one input element moves the 28-layer output by rel-L2 {sens:.3g}")
            assert_stack_close(outs[2], ref, what=f"persistent 28 layers t={t}")
            assert_stack_close(outs[1], ref, what=f"per-op 28 layers t={t}")
            assert kvs[2].used == ctx0 + t + 1
        rows = slice(ctx0, ctx0 + steps)
        for l in (0, 13, 27):
            kr = kcs[l].reshape(NKV, cap, HD)
            vr = vcs[l].reshape(NKV, cap, HD)
            for mode in (2, 1):
                k2, v2 = kvs[mode].download(l)
                if l == 0:
                    # layer 0 of the first token sees identical inputs
                    assert np.array_equal(k2[:, ctx0], kr[:, ctx0]) and np.array_equal(v2[:, ctx0], vr[:, ctx0])
                _kv_rows_close(orc, k2, kr, rows, f"mode {mode} layer {l} K rows")
                _kv_rows_close(orc, v2, vr, rows, f"mode {mode} layer {l} V rows")
                # rows outside the appended span are untouched
                assert np.array_equal(k2[:, :ctx0], kr[:, :ctx0]) and not k2[:, ctx0 + steps:].any()
    finally:
        for m in models.values():
            m.free()
        for kv in kvs.values():
            kv.free()


def test_prefill_512_full_width_per_layer(vxm_ctx, orc, stack28):
    """512-token causal prefill at full width, layer by layer for the first three
    layers: each device block against the oracle's block fed the same input, and
    the 512 K / V rows it writes."""
    import vxm

    layers, fn = stack28
    M, cap, n = 512, 512, 3
    rng = np.random.default_rng(512)
    c = cfg_dict(H, n, NH, NKV, HD, F)
    oc = orc_cfg(orc, c)
    m = vxm.MiniCPM4(vxm_ctx, c, layers[:n])
    kv = vxm.KVCache(vxm_ctx, n, NKV, HD, cap)
    try:
        x = rng.normal(0, 1, (M, H)).astype(np.float32)
        xd = _dev(x)
        for l in range(n):
            x_in = xd.cpu().numpy()
            m.block(kv, l, xd, 0)
            vxm_ctx.sync()
            kc = np.zeros(NKV * cap * HD, np.uint16)
            vc = np.zeros_like(kc)
            ref = orc.minicpm4_block(oc, to_orc(orc, layers[l]), x_in, kc, vc, cap, 0, 0)
            assert_layer_close(xd.cpu().numpy(), ref, frac=0.99, what=f"prefill 512 layer {l}")
            k2, v2 = kv.download(l)
            for got, want, nm in ((k2, kc, "K"), (v2, vc, "V")):
                eq = _kv_rows_close(orc, got, want.reshape(NKV, cap, HD), slice(0, M), f"layer {l} {nm} rows",
                                    bar=1e-3)
                assert eq >= 0.99, (l, nm, eq)
    finally:
        m.free()
        kv.free()


def test_prefill_512_28_layers_matches_oracle(vxm_ctx, orc, stack28):
    """The 512-token, 28-layer prefill workload in one call against the oracle's
    28-layer forward, with the KV rows of layers 0, 13 and 27."""
    import vxm

    layers, fn = stack28
    M, cap = 512, 512
    rng = np.random.default_rng(5120)
    c = cfg_dict(H, L, NH, NKV, HD, F)
    oc = orc_cfg(orc, c)
    m = vxm.MiniCPM4(vxm_ctx, c, layers, final_norm=fn)
    kv = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
    try:
        x = rng.normal(0, 1, (M, H)).astype(np.float32)
        xd = _dev(x)
        m.forward(kv, xd, 0)
        vxm_ctx.sync()
        assert kv.used == M
        kcs = [np.zeros(NKV * cap * HD, np.uint16) for _ in range(L)]
        vcs = [np.zeros(NKV * cap * HD, np.uint16) for _ in range(L)]
        ref = orc.minicpm4_forward(oc, [to_orc(orc, d) for d in layers], fn, x, kcs, vcs, cap, 0)
        assert_stack_close(xd.cpu().numpy(), ref, what="prefill 512 x 28 layers")
        for l in (0, 13, 27):
            k2, v2 = kv.download(l)
            _kv_rows_close(orc, k2, kcs[l].reshape(NKV, cap, HD), slice(0, M), f"prefill layer {l} K rows")
            _kv_rows_close(orc, v2, vcs[l].reshape(NKV, cap, HD), slice(0, M), f"prefill layer {l} V rows")
    finally:
        m.free()
        kv.free()


def test_prefill_512_equals_two_chunks_of_256(vxm_ctx, orc, stack28):
    """Prompt prefill in one 512-token call against 256 tokens then 256 more at
    position 256 (gen_prompt_eval_range over segments), 28 layers: outputs and
    the KV rows of layers 0, 13 and 27 agree to the stack bar."""
    import vxm

    layers, fn = stack28
    M, cap = 512, 512
    rng = np.random.default_rng(256)
    c = cfg_dict(H, L, NH, NKV, HD, F)
    m = vxm.MiniCPM4(vxm_ctx, c, layers, final_norm=fn)
    kva = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
    kvb = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
    try:
        x = rng.normal(0, 1, (M, H)).astype(np.float32)
        xa = _dev(x)
        m.forward(kva, xa, 0)
        xb0, xb1 = _dev(x[:256]), _dev(x[256:])
        m.forward(kvb, xb0, 0)
        m.forward(kvb, xb1, 256)
        vxm_ctx.sync()
        assert kva.used == M and kvb.used == M
        ya = xa.cpu().numpy()
        yb = np.concatenate([xb0.cpu().numpy(), xb1.cpu().numpy()])
        assert_stack_close(yb, ya, what="prefill 256 + 256 vs 512")
        for l in (0, 13, 27):
            ka, va = kva.download(l)
            kb, vb = kvb.download(l)
            _kv_rows_close(orc, kb, ka, slice(0, M), f"chunked layer {l} K rows")
            _kv_rows_close(orc, vb, va, slice(0, M), f"chunked layer {l} V rows")
    finally:
        m.free()
        kva.free()
        kvb.free()
