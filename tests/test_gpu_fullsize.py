"""GPU parity at the measured workloads' full sizes, against the oracle.

The MiniCPM4 TSLM shape (hidden 2048, 16 q / 2 kv heads of 128, SwiGLU 6144,
Q8_0 weights ~ N(0, 0.02)) at full depth (28 layers):
  * the 28-layer decode of consecutive tokens from context 256 on the
    single-launch (persistent) kernel and on the one-kernel-per-op path
    (vcpm_minicpm4_forward with n_tokens = 1, src/minicpm4.c:536-572), with
    the appended KV rows of the first, a middle and the last layer; and every
    one of the 28 layers on its own, fed the device's own input (teacher
    forcing: each layer's arithmetic alone, no compounding);
  * the 512-token prompt prefill (the M = n_tokens GEMMs of
    gen_prompt_eval_range, src/gen_prompt.c:186-272): all 28 layers teacher
    forced with the 512 K / V rows each writes, the whole 28-layer stack in one
    call, and 512 tokens in one call against two chunks of 256.

Bars (the numbers are pinned on the CPU by test_oracle_sensitivity.py).  The
device and the oracle differ only in fp32 summation order; where that moves a
value across a BF16 rounding boundary, the flip re-quantizes a Q8_0 block and
spreads.  The oracle itself shows the size of one flip: one BF16 ulp on one
input element moves a full-width block's output by a relative L2 of 4e-3
(512-token prefill; causal attention carries it to every later token) or
5.6e-3 (decode), and the 28-layer decode output by 5.7e-2 (cosine 0.998).
Hence:
  * one layer, teacher forced: relative L2 <= 1e-2 and every element within
    2^-5 of its row's largest magnitude;
  * 28 layers: cosine >= 0.995 and relative L2 <= 0.1, with the oracle's own
    one-ulp sensitivity printed beside the device's deviation;
  * K / V rows written from identical inputs: >= 99% identical, relative L2
    <= 1e-3.
"""
import numpy as np
import pytest

from test_gpu_minicpm4 import _dev, cfg_dict, layer_stats, orc_cfg, to_orc

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, F, L = 2048, 16, 2, 128, 6144, 28
LAYER_REL, LAYER_ROW = 1e-2, 2.0 ** -5      # one layer fed identical inputs
STACK_COS, STACK_REL = 0.995, 0.1           # 28 layers
KV_EQ, KV_REL = 0.99, 1e-3                  # K / V rows from identical inputs
# A K / V element from identical inputs can differ only by the fp32 order of its
# projection's block terms: at most one BF16 ulp (2^-7 of the value) before the
# rotary pair mixes it into two elements of at most sqrt(2) times the row max,
# plus the f16 rounding of the cache
KV_ULP = 2.0 ** -6


def assert_one_layer(y, ref, what):
    y64, r64 = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    rel = float(np.linalg.norm(y64 - r64) / np.linalg.norm(r64))
    row = float((np.abs(y64 - r64) / np.abs(r64).max(axis=-1, keepdims=True)).max())
    print(f"{what}: rel-L2 {rel:.3g}, worst element / row max {row:.3g}, {layer_stats(y, ref)}")
    assert rel <= LAYER_REL and row <= LAYER_ROW, (what, rel, row)
    return rel


def assert_stack(y, ref, what):
    a, b = np.ravel(y).astype(np.float64), np.ravel(ref).astype(np.float64)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
    rel = float(np.linalg.norm(a - b) / np.linalg.norm(b))
    print(f"{what}: cos {cos:.6f}, rel-L2 {rel:.3g}")
    assert cos >= STACK_COS and rel <= STACK_REL, (what, cos, rel)


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


def _kv_rel(orc, got_bits, want_bits, rows, what):
    g = orc.fp16_bits_to_fp32(got_bits)[:, rows].astype(np.float64)
    w = orc.fp16_bits_to_fp32(want_bits)[:, rows].astype(np.float64)
    rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
    eq = float((got_bits[:, rows] == want_bits[:, rows]).mean())
    print(f"{what}: rel-L2 {rel:.3g}, identical {eq:.4f}")
    return rel, eq


def _kv_worst(orc, got_bits, want_bits, rows):
    """Largest |got - want| over each head's row, relative to the row's max |want|."""
    g = orc.fp16_bits_to_fp32(got_bits)[:, rows].astype(np.float64)
    w = orc.fp16_bits_to_fp32(want_bits)[:, rows].astype(np.float64)
    return float((np.abs(g - w) / np.abs(w).max(axis=-1, keepdims=True)).max())


def _oracle_sensitivity(orc, oc, ol, fn, x, kcs, vcs, cap, pos, ref):
    """How far the oracle's own output moves when one input element moves by one
    BF16 ulp (printed beside the device's deviation)."""
    xp = x.copy()
    xp.flat[7] = np.float32(xp.flat[7] * (1 + 2.0 ** -7))
    alt = orc.minicpm4_forward(oc, ol, fn, xp, [k.copy() for k in kcs], [v.copy() for v in vcs], cap, pos)
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
            kc0, vc0 = [k.copy() for k in kcs], [v.copy() for v in vcs]
            ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0 + t)
            if t == 0:
                sens = _oracle_sensitivity(orc, oc, ol, fn, x, kc0, vc0, cap, ctx0, ref)
                print(f"oracle: one BF16 ulp on one input element moves its 28-layer output by rel-L2 {sens:.3g}")
            assert_stack(outs[2], ref, f"persistent 28 layers t={t}")
            assert_stack(outs[1], ref, f"per-op 28 layers t={t}")
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
                for got, want, nm in ((k2, kr, "K"), (v2, vr, "V")):
                    rel, _ = _kv_rel(orc, got, want, rows, f"mode {mode} layer {l} {nm} rows")
                    assert rel <= STACK_REL, (mode, l, nm, rel)
                # rows outside the appended span are untouched
                assert np.array_equal(k2[:, :ctx0], kr[:, :ctx0]) and not k2[:, ctx0 + steps:].any()
    finally:
        for m in models.values():
            m.free()
        for kv in kvs.values():
            kv.free()


def test_decode_every_layer_teacher_forced(vxm_ctx, orc, stack28):
    """Each of the 28 layers alone at the decode shape (context 256), on the
    single-launch kernel and on the per-op path: layer l is fed the persistent
    path's output of layer l - 1, and the oracle's block the same input and the
    same prior cache; the appended K / V row is compared as well."""
    import vxm

    layers, _ = stack28
    cap, ctx0 = 512, 256
    rng = np.random.default_rng(404)
    c = cfg_dict(H, 1, NH, NKV, HD, F)
    oc = orc_cfg(orc, c)
    x = rng.normal(0, 1, (1, H)).astype(np.float32)
    worst, exact = 0.0, 0
    for l in range(L):
        k, v = _prior_cache(orc, rng, cap, ctx0)
        outs, kvrows = {}, {}
        for mode in (2, 1):
            m = vxm.MiniCPM4(vxm_ctx, c, [layers[l]])
            m.set_decode_mode(mode)
            kv = vxm.KVCache(vxm_ctx, 1, NKV, HD, cap)
            try:
                kv.upload(0, k, v)
                xd = _dev(x)
                m.forward(kv, xd, ctx0)
                vxm_ctx.sync()
                m.check()
                outs[mode] = xd.cpu().numpy()
                kvrows[mode] = kv.download(0)
            finally:
                m.free()
                kv.free()
        kc, vc = k.reshape(-1).copy(), v.reshape(-1).copy()
        ref = orc.minicpm4_block(oc, to_orc(orc, layers[l]), x, kc, vc, cap, ctx0, 0)
        for mode in (2, 1):
            rel = assert_one_layer(outs[mode], ref, f"layer {l} mode {mode}")
            worst = max(worst, rel)
            exact += rel == 0.0
            # the appended row comes from identical inputs: only the projection's fp32 order differs
            for got, want, nm in ((kvrows[mode][0], kc, "K"), (kvrows[mode][1], vc, "V")):
                rows = slice(ctx0, ctx0 + 1)
                rel_kv, eq = _kv_rel(orc, got, want.reshape(NKV, cap, HD), rows, f"layer {l} mode {mode} {nm} row")
                worst_kv = _kv_worst(orc, got, want.reshape(NKV, cap, HD), rows)
                assert worst_kv <= KV_ULP and eq >= KV_EQ - 0.02, (l, mode, nm, rel_kv, worst_kv, eq)
                assert np.array_equal(got[:, :ctx0], want.reshape(NKV, cap, HD)[:, :ctx0])
        x = outs[2]
    print(f"28 layers x 2 paths: worst rel-L2 {worst:.3g}, {exact} of 56 bit-identical")


def test_prefill_512_every_layer_teacher_forced(vxm_ctx, orc, stack28):
    """The 512-token causal prefill at full width, each of the 28 layers fed the
    device's output of the previous layer: every device block against the
    oracle's block on the same input, and the 512 K / V rows it writes."""
    import vxm

    layers, _ = stack28
    M, cap = 512, 512
    rng = np.random.default_rng(512)
    c = cfg_dict(H, L, NH, NKV, HD, F)
    oc = orc_cfg(orc, c)
    m = vxm.MiniCPM4(vxm_ctx, c, layers)
    kv = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
    worst = 0.0
    try:
        xd = _dev(rng.normal(0, 1, (M, H)).astype(np.float32))
        for l in range(L):
            x_in = xd.cpu().numpy()
            m.block(kv, l, xd, 0)
            vxm_ctx.sync()
            kc = np.zeros(NKV * cap * HD, np.uint16)
            vc = np.zeros_like(kc)
            ref = orc.minicpm4_block(oc, to_orc(orc, layers[l]), x_in, kc, vc, cap, 0, 0)
            worst = max(worst, assert_one_layer(xd.cpu().numpy(), ref, f"prefill 512 layer {l}"))
            k2, v2 = kv.download(l)
            for got, want, nm in ((k2, kc, "K"), (v2, vc, "V")):
                rel, eq = _kv_rel(orc, got, want.reshape(NKV, cap, HD), slice(0, M), f"layer {l} {nm} rows")
                assert rel <= KV_REL and eq >= KV_EQ, (l, nm, rel, eq)
    finally:
        m.free()
        kv.free()
    print(f"28 prefill layers: worst rel-L2 {worst:.3g}")


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
        assert_stack(xd.cpu().numpy(), ref, "prefill 512 x 28 layers")
        for l in (0, 13, 27):
            k2, v2 = kv.download(l)
            for got, want, nm in ((k2, kcs[l], "K"), (v2, vcs[l], "V")):
                rel, eq = _kv_rel(orc, got, want.reshape(NKV, cap, HD), slice(0, M), f"prefill layer {l} {nm} rows")
                assert rel <= (KV_REL if l == 0 else STACK_REL), (l, nm, rel)
                if l == 0:
                    assert eq >= KV_EQ, (nm, eq)
    finally:
        m.free()
        kv.free()


def test_prefill_512_equals_two_chunks_of_256(vxm_ctx, orc, stack28):
    """Prompt prefill in one 512-token call against 256 tokens then 256 more at
    position 256 (gen_prompt_eval_range over segments), 28 layers: outputs and
    the KV rows of layers 0, 13 and 27 agree to the 28-layer bar; the first
    chunk's layer-0 K / V rows to the identical-input bar."""
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
        yb = np.concatenate([xb0.cpu().numpy(), xb1.cpu().numpy()])
        assert_stack(yb, xa.cpu().numpy(), "prefill 256 + 256 vs 512")
        for l in (0, 13, 27):
            ka, va = kva.download(l)
            kb, vb = kvb.download(l)
            for got, want, nm in ((kb, ka, "K"), (vb, va, "V")):
                rel, eq = _kv_rel(orc, got, want, slice(0, M), f"chunked layer {l} {nm} rows")
                assert rel <= STACK_REL, (l, nm, rel)
                if l == 0:
                    rel0, eq0 = _kv_rel(orc, got, want, slice(0, 256), f"chunked layer 0 {nm} rows of chunk 1")
                    assert rel0 <= KV_REL and eq0 >= KV_EQ, (nm, rel0, eq0)
    finally:
        m.free()
        kva.free()
        kvb.free()


@pytest.mark.parametrize("ctx0", [256, 700])
def test_decode_every_layer_of_one_28_layer_launch(vxm_ctx, orc, stack28, ctx0):
    """Depth inside ONE 28-layer single launch (and the per-op path): the library
    writes every layer's input and the last layer's output (vxm_minicpm4_set_layer_dump,
    the counterpart of the reference's per-node read-back), and the oracle's block l,
    fed the launch's own input to layer l and the same prior cache, must give the
    launch's input to layer l + 1 within the one-layer bar.  Layers 1-27 run on the
    code that a one-layer model never reaches (the two x buffers by layer parity,
    layer-table entries past 0, tags with layer bits, the ring across layer
    boundaries).  At 700 keys every head's keys are split over 3 workgroups, so the
    chunk merge is pinned at every depth too.  The K / V row each layer appends is
    compared with the oracle's from the same input."""
    import torch
    import vxm

    layers, fn = stack28
    cap = 1024
    rng = np.random.default_rng(505 + ctx0)
    c = cfg_dict(H, L, NH, NKV, HD, F)
    oc1 = orc_cfg(orc, cfg_dict(H, 1, NH, NKV, HD, F))
    caches = [_prior_cache(orc, rng, cap, ctx0) for _ in range(L)]
    x = rng.normal(0, 1, (1, H)).astype(np.float32)
    worst = 0.0
    for mode in (2, 1):
        m = vxm.MiniCPM4(vxm_ctx, c, layers, final_norm=fn)
        m.set_decode_mode(mode)
        kv = vxm.KVCache(vxm_ctx, L, NKV, HD, cap)
        dump = torch.full((L + 1, H), float("nan"), dtype=torch.float32, device="cuda:0")
        try:
            for l in range(L):
                kv.upload(l, *caches[l])
            m.set_layer_dump(dump)
            xd = _dev(x)
            print(f"28-layer decode with layer dump, mode {mode}, ctx {ctx0}", flush=True)
            m.forward(kv, xd, ctx0)
            vxm_ctx.sync()
            m.check()
            d = dump.cpu().numpy()
            out = xd.cpu().numpy()
            kvrows = [kv.download(l) for l in range(L)]
        finally:
            m.set_layer_dump(None)
            m.free()
            kv.free()
        assert np.isfinite(d).all(), "a layer's dump was not written"
        assert np.array_equal(d[0], x[0]), "layer 0's input is the call's x"
        # the returned row is the final norm of the last layer's output
        assert np.array_equal(out[0], orc.rms_norm(d[L:L + 1], fn, 1e-6)[0]), "final norm of the dumped output"
        for l in range(L):
            kc, vc = caches[l][0].reshape(-1).copy(), caches[l][1].reshape(-1).copy()
            ref = orc.minicpm4_block(oc1, to_orc(orc, layers[l]), d[l:l + 1], kc, vc, cap, ctx0, 0)
            worst = max(worst, assert_one_layer(d[l + 1:l + 2], ref, f"mode {mode} layer {l} of one launch"))
            rows = slice(ctx0, ctx0 + 1)
            for got, want, nm in ((kvrows[l][0], kc, "K"), (kvrows[l][1], vc, "V")):
                w3 = want.reshape(NKV, cap, HD)
                assert _kv_worst(orc, got, w3, rows) <= KV_ULP, (mode, l, nm)
    print(f"every layer of one launch, ctx {ctx0}: worst rel-L2 {worst:.3g}")
