"""GPU parity of the single-launch (persistent) decode against the oracle and
against the one-kernel-per-op path, at the MiniCPM4 TSLM / RALM shape (the
only shape the single-launch kernel is built for), with RoPE (LongRoPE
factors) and without (RALM), over consecutive tokens so the per-launch tags
and the KV append are exercised.  Other shapes take the per-op path.

Two last-ulp differences from the oracle are parity unpinned: the device's
cosf/sinf against glibc's (rope), and the persistent attention's score sum
(8-dim lane partials and a lane butterfly, where the oracle sums the head
dims in order; ggml's own F32 dot order depends on the host SIMD width).  A
one-ulp difference can move a value across a BF16 or Q8_0 rounding boundary,
which then spreads through every later op, so multi-step, multi-layer decode
outputs are held to a statistical bar: cosine >= 0.9995 and relative L2
error <= 2e-2 against the oracle.  The single-layer first-token case stays on
the strict per-element bar.
"""
import numpy as np
import pytest

from test_gpu_minicpm4 import _dev, assert_layer_close, cfg_dict, layer_stats, orc_cfg, rand_layer, to_orc


pytestmark = pytest.mark.gpu


def assert_stack_close(y, ref, what=""):
    s = layer_stats(y, ref)
    a = np.ravel(y).astype(np.float64)
    b = np.ravel(ref).astype(np.float64)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
    print(f"{what}: cos={cos:.6f} {s}")
    assert cos >= 0.9995 and s["rel_l2"] <= 2e-2, (what, cos, s)

SHAPES = {
    "tslm": dict(H=2048, nh=16, nkv=2, hd=128, F=6144),
    "small": dict(H=1024, nh=8, nkv=2, hd=128, F=2048),
}


def _setup(orc, vxm, vxm_ctx, shape, L, cap, ctx0, seed, no_rope=0, kscale=1.0):
    s = SHAPES[shape]
    rng = np.random.default_rng(seed)
    lws = [rand_layer(orc, rng, s["H"], s["nh"], s["nkv"], s["hd"], s["F"]) for _ in range(L)]
    fn = (1 + rng.normal(0, 0.02, s["H"])).astype(np.float32)
    c = cfg_dict(s["H"], L, s["nh"], s["nkv"], s["hd"], s["F"], no_rope=no_rope)
    models = {}
    for mode in (1, 2):
        m = vxm.MiniCPM4(vxm_ctx, c, lws, final_norm=fn)
        m.set_decode_mode(mode)
        models[mode] = m
    kvs = {mode: vxm.KVCache(vxm_ctx, L, s["nkv"], s["hd"], cap) for mode in (1, 2)}
    kcs, vcs = [], []
    for l in range(L):
        k = np.zeros((s["nkv"], cap, s["hd"]), np.uint16)
        v = np.zeros_like(k)
        k[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, kscale, (s["nkv"], ctx0, s["hd"])).astype(np.float32)))
        v[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (s["nkv"], ctx0, s["hd"])).astype(np.float32)))
        for mode in (1, 2):
            kvs[mode].upload(l, k, v)
        kcs.append(k.reshape(-1).copy())
        vcs.append(v.reshape(-1).copy())
    return s, rng, c, lws, fn, models, kvs, kcs, vcs


def test_persistent_first_token_single_layer_exact(vxm_ctx, orc):
    """One layer, first token: the persistent path matches the oracle on the
    strict per-element bar."""
    import vxm

    cap = 256
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", 1, cap, 100, 77)
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    xd = _dev(x)
    models[2].forward(kvs[2], xd, 100)
    vxm_ctx.sync()
    models[2].check()
    ref = orc.minicpm4_forward(orc_cfg(orc, c), [to_orc(orc, l) for l in lws], fn, x, kcs, vcs, cap, 100)
    assert_layer_close(xd.cpu().numpy(), ref, what="persistent 1 layer")
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


@pytest.mark.parametrize("shape,L,ctx0,steps,no_rope", [
    ("tslm", 3, 0, 3, 0),       # empty cache: the first tokens attend to themselves only
    ("tslm", 2, 200, 2, 1),     # the residual LM (RALM): no rope
    ("tslm", 2, 256, 3, 0),
    ("tslm", 1, 700, 2, 0),     # more keys than one attention batch
])
def test_persistent_decode_matches_oracle(vxm_ctx, orc, shape, L, ctx0, steps, no_rope):
    import vxm

    cap = 1024
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, shape, L, cap, ctx0, 31 + L + ctx0,
                                                       no_rope)
    oc = orc_cfg(orc, c)
    ol = [to_orc(orc, l) for l in lws]
    for t in range(steps):
        x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
        outs = {}
        for mode in (1, 2):
            xd = _dev(x)
            models[mode].forward(kvs[mode], xd, ctx0 + t)
            vxm_ctx.sync()
            outs[mode] = xd.cpu().numpy()
        models[2].check()
        ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0 + t)
        assert_stack_close(outs[2], ref, what=f"persistent {shape} t={t}")
        assert_stack_close(outs[1], ref, what=f"kernels {shape} t={t}")
        assert kvs[2].used == ctx0 + t + 1
    # the KV rows appended by both paths agree with the oracle's
    for l in range(L):
        k2, v2 = kvs[2].download(l)
        kr = orc.fp16_bits_to_fp32(kcs[l]).reshape(k2.shape)
        rows = slice(ctx0, ctx0 + steps)
        gk = orc.fp16_bits_to_fp32(k2)[:, rows]
        gv = orc.fp16_bits_to_fp32(v2)[:, rows]
        vr = orc.fp16_bits_to_fp32(vcs[l]).reshape(v2.shape)[:, rows]
        for got, want in ((gk, kr[:, rows]), (gv, vr)):
            if l == 0:
                # layer 0 of the first token sees identical inputs: exact rows
                assert np.array_equal(got[:, 0], want[:, 0])
            rel = np.linalg.norm(got - want) / np.linalg.norm(want)
            assert rel <= 2e-2, (l, rel)
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


def test_persistent_decode_repeatable(vxm_ctx, orc):
    """Same token at the same position twice gives bit-identical output (the
    dataflow tags, not timing, decide what each workgroup reads)."""
    import vxm

    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", 2, 256, 40, 5)
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    outs = []
    for _ in range(3):
        xd = _dev(x)
        models[2].forward(kvs[2], xd, 40)
        vxm_ctx.sync()
        outs.append(xd.cpu().numpy())
    models[2].check()
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


def test_persistent_unsupported_shape_falls_back(vxm_ctx, orc):
    """A shape without a single-launch kernel: AUTO decodes on the per-op path
    (still matching the oracle), PERSISTENT is refused with NOT_IMPLEMENTED."""
    import vxm

    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "small", 1, 256, 16, 9)
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    m_auto = vxm.MiniCPM4(vxm_ctx, c, lws, final_norm=fn)   # decode mode AUTO
    xd = _dev(x)
    m_auto.forward(kvs[1], xd, 16)
    vxm_ctx.sync()
    ref = orc.minicpm4_forward(orc_cfg(orc, c), [to_orc(orc, l) for l in lws], fn, x, kcs, vcs, 256, 16)
    assert_stack_close(xd.cpu().numpy(), ref, what="auto small")
    with pytest.raises(vxm.VxmError) as e:
        models[2].forward(kvs[2], _dev(x), 16)
    assert e.value.code == 7   # VXM_ERR_NOT_IMPLEMENTED
    m_auto.free()
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


def test_persistent_decode_after_cache_free_and_recreate(vxm_ctx, orc):
    """One model decodes on cache A (capacity 256), A is freed, and a new cache B
    of capacity 1024 is created (the allocator may hand B the struct address A
    had): the decode on B must read and append B's rows, not A's."""
    import vxm

    s = SHAPES["tslm"]
    L, ctx0 = 2, 100
    rng = np.random.default_rng(2024)
    lws = [rand_layer(orc, rng, s["H"], s["nh"], s["nkv"], s["hd"], s["F"]) for _ in range(L)]
    fn = (1 + rng.normal(0, 0.02, s["H"])).astype(np.float32)
    c = cfg_dict(s["H"], L, s["nh"], s["nkv"], s["hd"], s["F"])
    m = vxm.MiniCPM4(vxm_ctx, c, lws, final_norm=fn)
    m.set_decode_mode(2)
    oc, ol = orc_cfg(orc, c), [to_orc(orc, l) for l in lws]
    try:
        for cap in (256, 1024, 256):
            kv = vxm.KVCache(vxm_ctx, L, s["nkv"], s["hd"], cap)
            kcs, vcs = [], []
            for l in range(L):
                k = np.zeros((s["nkv"], cap, s["hd"]), np.uint16)
                v = np.zeros_like(k)
                k[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (s["nkv"], ctx0, s["hd"])).astype(np.float32)))
                v[:, :ctx0] = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (s["nkv"], ctx0, s["hd"])).astype(np.float32)))
                kv.upload(l, k, v)
                kcs.append(k.reshape(-1).copy())
                vcs.append(v.reshape(-1).copy())
            x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
            xd = _dev(x)
            m.forward(kv, xd, ctx0)
            vxm_ctx.sync()
            m.check()
            ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0)
            assert_stack_close(xd.cpu().numpy(), ref, what=f"cache of capacity {cap}")
            k0, v0 = kv.download(0)
            # layer 0 sees identical inputs: its appended row is exact, and nothing else moved
            assert np.array_equal(k0, kcs[0].reshape(k0.shape)) and np.array_equal(v0, vcs[0].reshape(v0.shape))
            kv.free()
    finally:
        m.free()


@pytest.mark.parametrize("ctx0,steps", [
    (382, 4),     # 383, 384 keys on one workgroup per head, then 385, 386 split in two chunks
    (2047, 2),    # 2048 keys: 8 chunks per head, 2049: 9
    (4095, 2),    # 4096 keys: 16 chunks of 256, 4097: 16 of 257
    (8190, 2),    # 8191, 8192 keys: 16 chunks of 512
])
def test_persistent_long_context_matches_oracle(vxm_ctx, orc, ctx0, steps):
    """Long contexts stay on the single-launch kernel, which splits each head's keys
    over up to 16 workgroups and merges the chunk softmaxes in chunk order: two
    full-width layers against the oracle and the per-op path, appended KV rows too."""
    import vxm

    cap, L = 8192, 2
    print(f"long context ctx0={ctx0} steps={steps}", flush=True)
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", L, cap, ctx0, 17 + ctx0)
    oc = orc_cfg(orc, c)
    ol = [to_orc(orc, l) for l in lws]
    for t in range(steps):
        x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
        outs = {}
        for mode in (1, 2):
            xd = _dev(x)
            models[mode].forward(kvs[mode], xd, ctx0 + t)
            vxm_ctx.sync()
            outs[mode] = xd.cpu().numpy()
        models[2].check()
        ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0 + t)
        assert_stack_close(outs[2], ref, what=f"persistent ctx {ctx0 + t + 1} keys")
        assert_stack_close(outs[1], ref, what=f"kernels ctx {ctx0 + t + 1} keys")
    for l in range(L):
        k2, v2 = kvs[2].download(l)
        rows = slice(ctx0, ctx0 + steps)
        for got, want in ((k2, kcs[l]), (v2, vcs[l])):
            g = orc.fp16_bits_to_fp32(got)[:, rows]
            w = orc.fp16_bits_to_fp32(want).reshape(got.shape)[:, rows]
            if l == 0:
                assert np.array_equal(g[:, 0], w[:, 0])
            assert np.linalg.norm(g - w) / np.linalg.norm(w) <= 2e-2
        # rows before ctx0 are untouched
        assert np.array_equal(k2[:, :ctx0], kcs[l].reshape(k2.shape)[:, :ctx0])
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


def test_persistent_long_context_repeatable(vxm_ctx, orc):
    """The chunk merge adds in chunk order: the same token at 4096 keys twice is
    bit-identical."""
    import vxm

    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", 2, 4200, 4095, 6)
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    outs = []
    for _ in range(3):
        xd = _dev(x)
        models[2].forward(kvs[2], xd, 4095)
        vxm_ctx.sync()
        outs.append(xd.cpu().numpy())
    models[2].check()
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


@pytest.mark.parametrize("ctx0", [384, 2047, 4095, 8191])
def test_persistent_long_context_peaked_attention(vxm_ctx, orc, ctx0):
    """One full-width layer at long context with keys of standard deviation 6: each
    head's softmax is dominated by a few keys and the attention output is as large as
    the residual, so the attention, and the merge of its key chunks, shows in the
    layer output.  The single-launch kernel sums a score's 128 products in another
    fp32 order than the oracle (parity unpinned), and with outputs this large one ulp
    can flip a Q8_0 or BF16 rounding that the rest of the layer spreads (a build that
    never splits the keys gives the same output at 2048 keys), so the bar is the
    stack bar.  Planted in the oracle on the CPU, an attention that loses its output
    (V = 0) or weights the chunks past the first wrongly (their V doubled) misses
    that bar many times over."""
    import vxm
    from test_gpu_minicpm4 import layer_stats

    cap, L = 8192, 1
    print(f"peaked attention ctx0={ctx0}", flush=True)
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", L, cap, ctx0, 91 + ctx0, kscale=6.0)
    oc, ol = orc_cfg(orc, c), [to_orc(orc, l) for l in lws]
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    xd = _dev(x)
    models[2].forward(kvs[2], xd, ctx0)
    vxm_ctx.sync()
    models[2].check()
    got = xd.cpu().numpy()
    k0, v0 = kcs[0].copy(), vcs[0].copy()
    ref = orc.minicpm4_forward(oc, ol, fn, x, kcs, vcs, cap, ctx0)
    assert_stack_close(got, ref, what=f"persistent 1 layer, {ctx0 + 1} keys")

    kv_len = ctx0 + 1
    n = 1 if kv_len <= 384 else min(16, (kv_len + 255) // 256)
    chl = (kv_len + n - 1) // n
    v_bad = orc.fp16_bits_to_fp32(v0).reshape(s["nkv"], cap, s["hd"])
    v_bad[:, chl:ctx0] *= 2.0
    plants = {"V = 0": np.zeros_like(v0),
              "V doubled past the first chunk": orc.fp32_to_fp16_bits(v_bad.astype(np.float32)).reshape(-1)}
    for what, vp in plants.items():
        bad = orc.minicpm4_forward(oc, ol, fn, x, [k0.copy()], [vp], cap, ctx0)
        st = layer_stats(got, bad)
        print(f"planted {what}: {st}")
        assert st["rel_l2"] >= 0.1, (what, st)   # the stack bar is rel_l2 <= 2e-2
    for m in models.values():
        m.free()
    for kv in kvs.values():
        kv.free()


def test_persistent_decode_two_streams_interleaved(vxm_ctx, orc):
    """Single-launch decodes from two contexts (two streams) of one device, issued
    alternately with no host synchronisation: each launch needs all 256 workgroups
    resident, and the library orders decode launches on a device across streams, so
    both sequences complete and equal their runs one token at a time bit for bit."""
    import vxm

    s = SHAPES["tslm"]
    L, cap, ctx0, steps = 2, 256, 50, 3
    rng = np.random.default_rng(777)
    lws = [rand_layer(orc, rng, s["H"], s["nh"], s["nkv"], s["hd"], s["F"]) for _ in range(L)]
    fn = (1 + rng.normal(0, 0.02, s["H"])).astype(np.float32)
    c = cfg_dict(s["H"], L, s["nh"], s["nkv"], s["hd"], s["F"])
    xs = [[rng.normal(0, 1, (1, s["H"])).astype(np.float32) for _ in range(steps)] for _ in range(2)]
    kh = orc.fp32_to_fp16_bits(orc.bf16_round(rng.normal(0, 1, (s["nkv"], cap, s["hd"])).astype(np.float32)))
    ctx2 = vxm.Context(0)
    contexts = (vxm_ctx, ctx2)

    def setup():
        ms, kvs = [], []
        for cx in contexts:
            m = vxm.MiniCPM4(cx, c, lws, final_norm=fn)
            m.set_decode_mode(2)
            kv = vxm.KVCache(cx, L, s["nkv"], s["hd"], cap)
            for l in range(L):
                kv.upload(l, kh, kh)
            kv.set_used(ctx0)
            ms.append(m)
            kvs.append(kv)
        return ms, kvs

    def teardown(ms, kvs):
        for m in ms:
            m.check()
            m.free()
        for kv in kvs:
            kv.free()

    try:
        # interleaved: token t of stream 0, token t of stream 1, ... no host sync
        ms, kvs = setup()
        dev = {}
        for t in range(steps):
            for j in range(2):
                xd = _dev(xs[j][t])
                ms[j].forward(kvs[j], xd, ctx0 + t)
                dev[(j, t)] = xd
        for cx in contexts:
            cx.sync()
        both = {k: v.cpu().numpy() for k, v in dev.items()}
        teardown(ms, kvs)
        # one token at a time, synchronised after each
        ms, kvs = setup()
        for j in range(2):
            for t in range(steps):
                xd = _dev(xs[j][t])
                ms[j].forward(kvs[j], xd, ctx0 + t)
                contexts[j].sync()
                assert np.array_equal(xd.cpu().numpy(), both[(j, t)]), (j, t)
        teardown(ms, kvs)
    finally:
        ctx2.close()


def test_persistent_decode_epoch_wrap(vxm_ctx, orc):
    """The single-launch decode tags its exchanged words with a 20-bit epoch kept in
    device memory.  Across the wrap (2^20 - 1 -> 1) the launch that wraps resets every
    exchange word, so a word from before the wrap cannot carry a live tag again.  The
    hazard is a key-chunk partial: chunk slots 2 and 3 of every head are written only
    by launches that split the keys 4 ways.  Here the first launch (epoch 1) splits
    1001 keys 4 ways; the launches just below the wrap split 501 keys 2 ways (slots 2
    and 3 keep their epoch-1 words); the launch after the wrap runs with epoch 1 again
    on 1001 keys and a new token.  Every output is held to the oracle."""
    import vxm

    L, cap = 2, 2048
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", L, cap, 1000, 606)
    m, kv = models[2], kvs[2]
    oc = orc_cfg(orc, c)
    ol = [to_orc(orc, l) for l in lws]
    base_k = [k.copy() for k in kcs]
    base_v = [v.copy() for v in vcs]
    shp = (s["nkv"], cap, s["hd"])

    def decode(pos, what):
        # the same prior cache every time (rows up to pos from the host)
        for l in range(L):
            kv.upload(l, base_k[l].reshape(shp), base_v[l].reshape(shp))
        x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
        xd = _dev(x)
        print(f"epoch wrap: {what} at pos {pos}", flush=True)
        m.forward(kv, xd, pos)
        vxm_ctx.sync()
        m.check()
        ref = orc.minicpm4_forward(oc, ol, fn, x, [k.copy() for k in base_k], [v.copy() for v in base_v], cap, pos)
        assert_stack_close(xd.cpu().numpy(), ref, what=what)

    try:
        decode(1000, "epoch 1, 4 key chunks")
        assert m.decode_epoch() == 2
        m.set_decode_epoch(0xFFFFE)
        decode(500, "epoch 0xffffe, 2 key chunks")
        decode(500, "epoch 0xfffff, 2 key chunks (wraps)")
        assert m.decode_epoch() == 1, "the wrap skips epoch 0"
        decode(1000, "epoch 1 after the wrap, 4 key chunks")
        decode(1000, "epoch 2 after the wrap")
        assert m.decode_epoch() == 3
        with pytest.raises(vxm.VxmError):
            m.set_decode_epoch(0)
        with pytest.raises(vxm.VxmError):
            m.set_decode_epoch(1 << 20)
    finally:
        for mm in models.values():
            mm.free()
        for k in kvs.values():
            k.free()


def test_single_launch_kernels_on_two_streams(vxm_ctx, orc):
    """A single-launch decode and a single-launch LocDiT evaluation issued from two
    contexts (two streams of one device) with no host synchronisation in between:
    every eager single-launch kernel is ordered after the device's previous one, so
    neither interleaves its workgroups with the other, and each result is
    bit-identical to the same call run alone."""
    import torch
    import vxm
    from locdit_case import make_inputs, make_locdit

    cap = 512
    s, rng, c, lws, fn, models, kvs, kcs, vcs = _setup(orc, vxm, vxm_ctx, "tslm", 2, cap, 300, 707)
    dm, dkv = models[2], kvs[2]
    shp = (s["nkv"], cap, s["hd"])
    base = [(k.copy(), v.copy()) for k, v in zip(kcs, vcs)]
    x = rng.normal(0, 1, (1, s["H"])).astype(np.float32)
    ctx2 = vxm.Context(0)
    cfg, w, ow, ocfg = make_locdit(orc, 808, 1024, 3, 16, 2, 128, 4096, 64, True)
    ld = vxm.LocDiT(ctx2, cfg, w)
    ld.set_block_mode(vxm.DECODE_PERSISTENT)
    lx, lcond, lmu = make_inputs(809, 4, 4, 64, 1024)

    def run_decode():
        for l in range(2):
            dkv.upload(l, base[l][0].reshape(shp), base[l][1].reshape(shp))
        xd = _dev(x)
        dm.forward(dkv, xd, 300)
        return xd

    def run_locdit():
        return ld.forward(_dev(lx), _dev(lcond), 0.4, 0.0, _dev(lmu))

    try:
        alone_d = run_decode()
        vxm_ctx.sync()
        alone_d = alone_d.cpu().numpy()
        alone_l = run_locdit()
        ctx2.sync()
        alone_l = alone_l.cpu().numpy()
        torch.cuda.synchronize()
        for rep in range(3):
            print(f"two streams, round {rep}", flush=True)
            yd = run_decode()
            yl = run_locdit()       # other context, other stream, no sync in between
            yd2 = run_decode() if rep == 2 else None
            vxm_ctx.sync()
            ctx2.sync()
            dm.check()
            ld.check()
            assert np.array_equal(yd.cpu().numpy(), alone_d), f"decode differs in round {rep}"
            assert np.array_equal(yl.cpu().numpy(), alone_l), f"locdit differs in round {rep}"
            if yd2 is not None:
                assert np.array_equal(yd2.cpu().numpy(), alone_d)
    finally:
        ld.free()
        ctx2.close()
        for mm in models.values():
            mm.free()
        for k in kvs.values():
            k.free()
