"""GPU parity of LocEnc, the FSQ core and the per-token LM update against the oracle.

FSQ (vcpm_fsq_quantize): the device's tanhf and the C library's may differ in
the last bit, so an output is compared bit for bit wherever tanh(x) * s is
more than 4 ulps away from a rounding tie (the rest is parity unpinned at
one grid step).

LocEnc outputs pass through the blocks' BF16 rounds and carry the block bar
(>= 99.5% of elements within 1e-3 rel / 1e-4 abs, <= 4 BF16 ulps, rel-L2
<= 1e-3).  The full-size encoder (12 bidirectional blocks) is compared block
by block, each device block fed the oracle's input to it, against the
re-quantization sensitivity bar of the LocDiT blocks (rel-L2 < 5e-3, every
element within 2^-6 of its row's scale), with a gross bar end to end.

The LM update is checked stage by stage: each device stage's output against
the oracle's stage fed the DEVICE's previous stage output and the device's KV
caches, so differences do not compound across stages; FSQ rounding ties are
excluded by checking that every element of the oracle's pre-round values is
at least 1e-3 away from one (a seeded precondition).  Multi-layer decode
stages take the decode bars (block bar per layer; cos >= 0.9995 and rel-L2
<= 2e-2 for stacks), end-to-end chains a gross bar.
"""
import numpy as np
import pytest

from test_gpu_decode import assert_stack_close
from test_gpu_locdit import assert_sensitivity_close
from test_gpu_minicpm4 import _dev, assert_layer_close
from test_lm_update_host import make_locenc, make_lm_update

pytestmark = pytest.mark.gpu


def _np(t):
    return t.cpu().numpy()


def _near_tie(v, s):
    v = np.abs(np.asarray(v, np.float64))
    return np.abs(v - np.floor(v) - 0.5) < 4 * np.spacing(np.float32(max(s, 1.0)))


@pytest.mark.parametrize("s", [9.0, 2.5, 0.0])
def test_fsq_quantize_matches_oracle(vxm_ctx, orc, s):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 50000), rng.normal(0, 4, 5000), [0, -0.0, 20, -20, 1e-30]])
    x = x.astype(np.float32)
    y = _np(vxm_ctx.fsq_quantize(_dev(x), s))
    ref = orc.fsq_quantize(x, s)
    # |x| >= 10: tanhf is exactly +-1 on both sides, so exact ties (s = 2.5) must round alike
    sat = np.abs(x) >= 10
    assert np.array_equal(y[sat], ref[sat])
    near = _near_tie(np.tanh(x.astype(np.float64)) * s, s) & ~sat if s > 0 else np.zeros(x.size, bool)
    # s = 2.5 puts a tie at saturation: for 7.5 < |x| < 10 one ulp of tanhf decides the rounding
    assert near.mean() < (0.06 if s == 2.5 else 0.001), near.mean()
    assert np.array_equal(y[~near], ref[~near]), np.nonzero(y[~near] != ref[~near])[0][:10]
    if s > 0:   # the rest differ by at most one grid step
        assert np.abs(y - ref).max() <= np.float32(1.0) / np.float32(s) * 1.0001


@pytest.mark.parametrize("special,bias", [(True, True), (False, True), (True, False)])
@pytest.mark.parametrize("P", [1, 4, 7])
def test_locenc_small(vxm_ctx, orc, special, bias, P):
    import vxm

    cfg, w, ow, ocfg = make_locenc(orc, 40 + P, special=special, bias=bias)
    x = np.random.default_rng(50 + P).normal(0, 1, (P, 64)).astype(np.float32)
    enc = vxm.LocEnc(vxm_ctx, cfg, w)
    out = _np(enc.forward(_dev(x)))
    ref = orc.locenc_forward(ocfg, ow, x)
    assert out.shape == ref.shape
    assert_layer_close(out, ref, what=f"locenc P={P} special={special} bias={bias}")
    enc.free()


def test_locenc_head_dim_128_rope_factors(vxm_ctx, orc):
    """head_dim 128 takes the LongRoPE short factors (the reference rule) on both sides."""
    import vxm

    cfg, w, ow, ocfg = make_locenc(orc, 61, H=256, L=2, nh=4, nkv=2, hd=128, F=512)
    x = np.random.default_rng(62).normal(0, 1, (4, 64)).astype(np.float32)
    enc = vxm.LocEnc(vxm_ctx, cfg, w)
    assert_layer_close(_np(enc.forward(_dev(x))), orc.locenc_forward(ocfg, ow, x), what="locenc hd=128")
    enc.free()


def test_locenc_full_size(vxm_ctx, orc):
    """The VoxCPM2 encoder: hidden 1024, 12 layers, 16 / 2 heads x 128, FFN 4096, one 4-position patch
    plus the special token.  Every block meets the sensitivity bar against the oracle's input to it."""
    import vxm

    cfg, w, ow, ocfg = make_locenc(orc, 71, H=1024, L=12, nh=16, nkv=2, hd=128, F=4096)
    x = np.random.default_rng(72).normal(0, 1, (4, 64)).astype(np.float32)
    enc = vxm.LocEnc(vxm_ctx, cfg, w)
    out = _np(enc.forward(_dev(x)))
    ref, states = orc.locenc_forward(ocfg, ow, x, states=True)
    blocks = vxm.MiniCPM4(vxm_ctx, dict(hidden_size=1024, n_layers=12, n_heads=16, n_kv_heads=2, head_dim=128,
                                        intermediate_size=4096, rms_norm_eps=1e-6, rope_theta=10000), w["layers"])
    for l in range(12):
        h = _dev(states[l])
        blocks.block(None, l, h, 0, 1)
        assert_sensitivity_close(_np(h), states[l + 1], what=f"locenc block {l}")
    blocks.free()
    rel = np.linalg.norm(out.astype(np.float64) - ref) / np.linalg.norm(ref)
    print(f"locenc end-to-end rel_l2 {rel:.3e}")
    assert np.isfinite(out).all() and rel < 5e-2
    enc.free()


def test_locenc_rejects_bad_sizes(vxm_ctx, orc):
    import vxm

    cfg, w, ow, ocfg = make_locenc(orc, 80)
    enc = vxm.LocEnc(vxm_ctx, cfg, w)
    with pytest.raises(vxm.VxmError):
        enc.forward(_dev(np.zeros((0, 64), np.float32)))
    enc.free()
    bad = dict(cfg, feat_dim=48)
    with pytest.raises(vxm.VxmError):
        vxm.LocEnc(vxm_ctx, bad, w)


def _device_lm(vxm, vxm_ctx, lm, cfg_kw):
    c = dict(cfg_kw)
    m = vxm.MiniCPM4(vxm_ctx, c, lm["dev"], final_norm=lm["norm"])
    kv = vxm.KVCache(vxm_ctx, c["n_layers"], c["n_kv_heads"], c["head_dim"], lm["cap"])
    return m, kv


def _sync_caches(kv, lm):
    """The oracle's caches := the device's (so a stage is checked on the device's own history)."""
    for l in range(len(lm["k"])):
        k, v = kv.download(l)
        lm["k"][l][...] = k
        lm["v"][l][...] = v


def _build_update(vxm, vxm_ctx, orc, seed, with_fsq, dims):
    enc, tslm, ralm, pw = make_lm_update(orc, seed, with_fsq=with_fsq, **dims["sizes"])
    ecfg, ew, eow, eocfg = enc
    e = vxm.LocEnc(vxm_ctx, ecfg, ew)
    tm, tkv = _device_lm(vxm, vxm_ctx, tslm, dims["tslm"])
    rm, rkv = _device_lm(vxm, vxm_ctx, ralm, dims["ralm"])
    w = dict(enc_to_lm=pw["enc_to_lm"], enc_to_lm_bias=pw["enc_to_lm_bias"], fusion_concat=pw["fusion"])
    if with_fsq:
        w.update(fsq_in=pw["fsq_in"], fsq_in_bias=pw["fsq_in_bias"], fsq_out=pw["fsq_out"],
                 fsq_out_bias=pw["fsq_out_bias"])
    s = dims["sizes"]
    u = vxm.LMUpdate(vxm_ctx, dict(lm_hidden=s["L"], enc_hidden=s["E"], fsq_dim=s["Fq"] if with_fsq else 0,
                                   res_hidden=s["R"], fsq_quant_scale=9.0), w, e, tm, rm)
    return (e, eow, eocfg), (tm, tkv, tslm), (rm, rkv, ralm), pw, u


def _check_update(orc, vxm_ctx, enc, tsl, ral, pw, u, steps, patch_seed, stack_bar, pos0=0):
    e, eow, eocfg = enc
    tm, tkv, tslm = tsl
    rm, rkv, ralm = ral
    L, E, R = pw["L"], pw["E"], pw["R"]
    rng = np.random.default_rng(patch_seed)
    for pos in range(pos0, pos0 + steps):
        patch = rng.normal(0, 1, (4, 64)).astype(np.float32)
        _sync_caches(tkv, tslm)
        _sync_caches(rkv, ralm)
        a, b, f, r = [_np(t) for t in u.step(tkv, rkv, _dev(patch), pos)]
        assert tkv.used == pos + 1 and rkv.used == pos + 1
        # audio embedding from the oracle encoder
        a_ref = orc.linear(pw["enc_to_lm"], orc.locenc_forward(eocfg, eow, patch), L, E, pw["enc_to_lm_bias"])[0]
        assert_layer_close(a, a_ref, what=f"pos {pos} audio_embed")
        # TSLM step on the device's audio embedding and caches
        b_ref = orc.minicpm4_forward(tslm["cfg"], tslm["layers"], tslm["norm"], a[None], tslm["k"], tslm["v"],
                                     tslm["cap"], pos)[0]
        stack_bar(b, b_ref, what=f"pos {pos} base_hidden")
        # FSQ on the device's TSLM hidden
        if pw.get("fsq_in") is not None:
            h = orc.linear(pw["fsq_in"], b, pw["Fq"], L, pw["fsq_in_bias"])[0]
            v = np.abs(np.tanh(h.astype(np.float64)) * 9.0)
            assert (np.abs(v - np.floor(v) - 0.5) > 1e-3).all(), "seeded case sits on an FSQ rounding tie"
            f_ref = orc.linear(pw["fsq_out"], orc.fsq_quantize(h, 9.0), L, pw["Fq"], pw["fsq_out_bias"])[0]
            assert_layer_close(f, f_ref, what=f"pos {pos} fsq")
        else:
            assert np.array_equal(f, b)
        # RALM step on the device's fusion input and caches
        ralm_in = orc.linear(pw["fusion"], np.concatenate([f, a]), R, 2 * L)[0]
        r_ref = orc.minicpm4_forward(ralm["cfg"], ralm["layers"], ralm["norm"], ralm_in[None], ralm["k"],
                                     ralm["v"], ralm["cap"], pos)[0]
        stack_bar(r, r_ref, what=f"pos {pos} ralm_hidden")


SMALL = dict(sizes=dict(L=128, E=128, Fq=64, R=128, cap=16),
             tslm=dict(hidden_size=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, intermediate_size=256,
                       rms_norm_eps=1e-6, rope_theta=10000, no_rope=0),
             ralm=dict(hidden_size=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, intermediate_size=256,
                       rms_norm_eps=1e-6, rope_theta=10000, no_rope=1))


@pytest.mark.parametrize("with_fsq", [True, False])
def test_lm_update_small_three_steps(vxm_ctx, orc, with_fsq):
    import vxm

    enc, tsl, ral, pw, u = _build_update(vxm, vxm_ctx, orc, 90, with_fsq, SMALL)

    def stack_bar(y, ref, what):
        assert_layer_close(y, ref, what=what)

    _check_update(orc, vxm_ctx, enc, tsl, ral, pw, u, 3, 91, stack_bar)
    u.free()
    for o in (enc[0], tsl[0], ral[0], tsl[1], ral[1]):
        o.free()


def test_lm_update_full_width_persistent(vxm_ctx, orc):
    """TSLM and RALM at the decode shape (hidden 2048, 16 / 2 heads x 128, FFN 6144; 2 layers each, the
    RALM without rope) run on the single-launch decode kernel inside the update; LocEnc at full width
    (1 block), FSQ 2048 -> 512 -> 2048, fusion 4096 -> 2048."""
    import vxm

    full = dict(sizes=dict(L=2048, E=1024, Fq=512, R=2048, cap=64,
                           enc_kw=dict(L=1, nh=16, nkv=2, hd=128, F=4096),
                           lm_kw=dict(n_layers=2, nh=16, nkv=2, hd=128, F=6144)),
                tslm=dict(hidden_size=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                          intermediate_size=6144, rms_norm_eps=1e-6, rope_theta=10000, no_rope=0),
                ralm=dict(hidden_size=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                          intermediate_size=6144, rms_norm_eps=1e-6, rope_theta=10000, no_rope=1))
    enc, tsl, ral, pw, u = _build_update(vxm, vxm_ctx, orc, 100, True, full)
    _check_update(orc, vxm_ctx, enc, tsl, ral, pw, u, 2, 101, assert_stack_close)
    u.free()
    for o in (enc[0], tsl[0], ral[0], tsl[1], ral[1]):
        o.free()


def _check_prompt(orc, tsl, ral, pw, u, x, pos, stack_bar, what):
    """gen_prompt_eval_range on the device, stage by stage: the base LM on x against the oracle's on the
    device's caches, the RALM on the device's own fusion input of [base ; 0]."""
    tm, tkv, tslm = tsl
    rm, rkv, ralm = ral
    L, R = pw["L"], pw["R"]
    n = x.shape[0]
    _sync_caches(tkv, tslm)
    _sync_caches(rkv, ralm)
    b, r = u.prompt_prefill(tkv, rkv, _dev(x), pos)
    b, r = _np(b), _np(r)
    assert b.shape == (n, L) and r.shape == (n, R)
    assert tkv.used == pos + n and rkv.used == pos + n
    b_ref = orc.minicpm4_forward(tslm["cfg"], tslm["layers"], tslm["norm"], x, tslm["k"], tslm["v"], tslm["cap"], pos)
    stack_bar(b, b_ref, what=f"{what} base_hidden")
    ralm_in = orc.linear(pw["fusion"], np.concatenate([b, np.zeros_like(b)], axis=1), R, 2 * L)
    r_ref = orc.minicpm4_forward(ralm["cfg"], ralm["layers"], ralm["norm"], ralm_in, ralm["k"], ralm["v"],
                                 ralm["cap"], pos)
    stack_bar(r, r_ref, what=f"{what} ralm_hidden")


def test_prompt_prefill_small_then_update(vxm_ctx, orc):
    """Prompt of 7 tokens in two ranges (gen_prompt_eval_range's pos_start), then two LM updates that
    attend to the prompt's cache rows."""
    import vxm

    small = dict(SMALL, sizes=dict(SMALL["sizes"], cap=24))
    enc, tsl, ral, pw, u = _build_update(vxm, vxm_ctx, orc, 110, True, small)
    x = np.random.default_rng(111).normal(0, 1, (7, 128)).astype(np.float32)

    def bar(y, ref, what):
        assert_layer_close(y, ref, what=what)

    _check_prompt(orc, tsl, ral, pw, u, x[:4], 0, bar, "prompt rows 0-3")
    _check_prompt(orc, tsl, ral, pw, u, x[4:], 4, bar, "prompt rows 4-6")
    _check_update(orc, vxm_ctx, enc, tsl, ral, pw, u, 2, 112, bar, pos0=7)
    u.free()
    for o in (enc[0], tsl[0], ral[0], tsl[1], ral[1]):
        o.free()


@pytest.mark.parametrize("n,chunks", [(40, 1), (96, 1), (160, 2)])
def test_prompt_prefill_full_width(vxm_ctx, orc, n, chunks):
    """The prompt prefill at the TSLM / RALM block shape (hidden 2048, 16 / 2 heads x 128, FFN 6144, 2 layers
    each, RALM without rope; fusion 4096 -> 2048): 40 tokens take the small-M GEMM, 96 and 80 the tiled MFMA
    GEMM and the MFMA attention."""
    import vxm

    full = dict(sizes=dict(L=2048, E=1024, Fq=512, R=2048, cap=192,
                           enc_kw=dict(L=1, nh=16, nkv=2, hd=128, F=4096),
                           lm_kw=dict(n_layers=2, nh=16, nkv=2, hd=128, F=6144)),
                tslm=dict(hidden_size=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                          intermediate_size=6144, rms_norm_eps=1e-6, rope_theta=10000, no_rope=0),
                ralm=dict(hidden_size=2048, n_layers=2, n_heads=16, n_kv_heads=2, head_dim=128,
                          intermediate_size=6144, rms_norm_eps=1e-6, rope_theta=10000, no_rope=1))
    print(f"prompt prefill full width n={n} chunks={chunks}", flush=True)
    enc, tsl, ral, pw, u = _build_update(vxm, vxm_ctx, orc, 120 + n, False, full)
    x = np.random.default_rng(121 + n).normal(0, 1, (n, 2048)).astype(np.float32)
    step = n // chunks
    for c in range(chunks):
        _check_prompt(orc, tsl, ral, pw, u, x[c * step:(c + 1) * step], c * step, assert_stack_close,
                      f"prompt rows {c * step}-{(c + 1) * step - 1}")
    u.free()
    for o in (enc[0], tsl[0], ral[0], tsl[1], ral[1]):
        o.free()


def test_embed_rows_q8_0_bit_exact(vxm_ctx, orc):
    """Q8_0 text-embedding rows gathered and dequantized on the device equal the oracle's, ids outside
    the table reading row 0."""
    import torch

    rng = np.random.default_rng(130)
    rows, k = 1000, 2048
    table = orc.quantize_rows(rng.normal(0, 0.05, (rows, k)).astype(np.float32), orc.QUANT_REF)
    w = vxm_ctx.upload_q8_0(table, rows, k)
    ids = np.array([5, 999, 0, -3, 1000, 123, 123, 77] + list(rng.integers(0, rows, 56)), np.int32)
    out = _np(vxm_ctx.embed_rows_q8_0(w, torch.from_numpy(ids).to("cuda:0")))
    assert np.array_equal(out, orc.embed_rows_q8_0(table, rows, k, ids))
    w.free()
