"""CPU pins of the oracle's LocEnc, FSQ and LM-update pieces (no GPU).

The FSQ core (vcpm_fsq_quantize, src/fsq.c:16-29) is pinned by closed forms
and known answers, including ggml_round's half-away-from-zero rule at exact
ties.  LocEnc (vcpm_locenc_forward, src/locenc.c:44-131) is pinned
structurally on top of the already pinned MiniCPM4 block and RMSNorm: with no
blocks the output is RMSNorm(special token) whatever x is; the first state is
[special ; in_proj x + bias] without a BF16 round; every state is the pinned
bidirectional block of the previous one; the output is the RMSNorm of the
last state's special row.  The LM update is a composition of pinned pieces;
its own checks cover the FSQ-less model and where the caches are written.
"""
import numpy as np
import pytest

from locdit_case import q8


def _layers(orc, rng, L, H, nh, nkv, hd, F):
    out, dev = [], []
    for _ in range(L):
        d = dict(q_proj=q8(orc, rng, nh * hd, H), k_proj=q8(orc, rng, nkv * hd, H), v_proj=q8(orc, rng, nkv * hd, H),
                 o_proj=q8(orc, rng, H, nh * hd), gate_proj=q8(orc, rng, F, H), up_proj=q8(orc, rng, F, H),
                 down_proj=q8(orc, rng, H, F),
                 input_layernorm=(1 + rng.normal(0, 0.02, H)).astype(np.float32),
                 post_attention_layernorm=(1 + rng.normal(0, 0.02, H)).astype(np.float32))
        dev.append(d)
        out.append(orc.LayerW(wq=d["q_proj"], wk=d["k_proj"], wv=d["v_proj"], wo=d["o_proj"], wg=d["gate_proj"],
                              wu=d["up_proj"], wd=d["down_proj"], g_in=d["input_layernorm"],
                              g_post=d["post_attention_layernorm"]))
    return out, dev


def make_locenc(orc, seed, H=128, L=2, nh=4, nkv=2, hd=32, F=256, feat=64, special=True, bias=True):
    """(device config, vxm weight dict, oracle LocEncW, oracle cfg) of a seeded LocEnc."""
    rng = np.random.default_rng(seed)
    lws, dev = _layers(orc, rng, L, H, nh, nkv, hd, F)
    w = dict(layers=dev, in_proj=q8(orc, rng, H, feat, 0.1),
             in_bias=rng.normal(0, 0.02, H).astype(np.float32) if bias else None,
             special_token=rng.normal(0, 1, H).astype(np.float32) if special else None,
             norm=(1 + rng.normal(0, 0.02, H)).astype(np.float32))
    cfg = dict(hidden_size=H, n_layers=L, n_heads=nh, n_kv_heads=nkv, head_dim=hd, intermediate_size=F,
               feat_dim=feat, rms_norm_eps=1e-6, rope_theta=10000)
    ow = orc.LocEncW(lws, feat, in_proj=w["in_proj"], in_bias=w["in_bias"], special=w["special_token"],
                     norm=w["norm"])
    ocfg = orc.make_cfg(H, nh, nkv, hd, F, eps=1e-6, rope_theta=10000.0,
                        rope_ff=orc.ROPE_SHORT_FACTORS if hd == 128 else None)
    return cfg, w, ow, ocfg


def _round_half_away(v):
    v = np.asarray(v, np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_fsq_known_answers(orc):
    # tanhf saturates to exactly +-1 at |x| = 20: round(+-9) * (1/9) = +-1
    y = orc.fsq_quantize(np.float32([0.0, -0.0, 20.0, -20.0]), 9.0)
    assert y[0] == 0 and y[1] == 0 and y[2] == np.float32(9) * np.float32(1 / np.float32(9)) and y[3] == -y[2]
    # exact ties: tanh = 1, s = 2.5 -> 2.5 rounds AWAY from zero to 3 (round-half-even would give 2)
    y = orc.fsq_quantize(np.float32([20.0, -20.0]), 2.5)
    inv = np.float32(1.0) / np.float32(2.5)
    assert y[0] == np.float32(3) * inv and y[1] == -np.float32(3) * inv
    y = orc.fsq_quantize(np.float32([20.0, -20.0]), 0.5)   # 0.5 -> 1, -0.5 -> -1
    assert y[0] == np.float32(2.0) and y[1] == np.float32(-2.0)
    # quant_scale <= 0 is the identity (src/fsq.c:19)
    x = np.random.default_rng(0).normal(0, 1, 64).astype(np.float32)
    assert np.array_equal(orc.fsq_quantize(x, 0.0), x) and np.array_equal(orc.fsq_quantize(x, -1.0), x)


def test_fsq_closed_form(orc):
    """y = round_half_away(tanh(x) s) * fl(1/s): the values are k * fl(1/s) with |k| <= round(s), and k matches
    numpy's tanh except where tanh(x) s sits within 4 ulps of a half-integer."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 4, 2000)]).astype(np.float32)
    for s in (9.0, 4.0, 1.5):
        y = orc.fsq_quantize(x, s)
        inv = np.float32(1.0) / np.float32(s)
        v = np.tanh(x).astype(np.float32) * np.float32(s)
        k = _round_half_away(v)
        assert np.abs(k).max() <= np.floor(s + 0.5)
        frac = np.abs(np.abs(v.astype(np.float64)) - np.floor(np.abs(v.astype(np.float64))) - 0.5)
        near = frac < 4 * np.spacing(np.float32(s))
        expect = (k.astype(np.float32) * inv).astype(np.float32)
        assert np.array_equal(y[~near], expect[~near]), s
        # every output is an integer multiple of fl(1/s)
        kk = y.astype(np.float64) / np.float64(inv)
        assert np.allclose(kk, np.round(kk), atol=1e-4)


def test_locenc_without_blocks_is_norm_of_special(orc):
    cfg, w, ow, ocfg = make_locenc(orc, 3, L=0)
    rng = np.random.default_rng(4)
    a = orc.locenc_forward(ocfg, ow, rng.normal(0, 1, (4, 64)).astype(np.float32))
    b = orc.locenc_forward(ocfg, ow, rng.normal(0, 1, (7, 64)).astype(np.float32))
    ref = orc.rms_norm(w["special_token"][None], w["norm"], 1e-6)[0]
    assert np.array_equal(a, ref) and np.array_equal(b, ref)


def test_locenc_without_special_token_returns_every_row(orc):
    cfg, w, ow, ocfg = make_locenc(orc, 5, L=0, special=False)
    x = np.random.default_rng(6).normal(0, 1, (3, 64)).astype(np.float32)
    out = orc.locenc_forward(ocfg, ow, x)
    h = orc.linear(w["in_proj"], x, 128, 64, w["in_bias"])
    assert out.shape == (3, 128)
    assert np.array_equal(out, orc.rms_norm(h, w["norm"], 1e-6))


@pytest.mark.parametrize("special", [True, False])
def test_locenc_states_chain_through_the_pinned_block(orc, special):
    cfg, w, ow, ocfg = make_locenc(orc, 7, L=2, special=special)
    x = np.random.default_rng(8).normal(0, 1, (4, 64)).astype(np.float32)
    out, st = orc.locenc_forward(ocfg, ow, x, states=True)
    h = orc.linear(w["in_proj"], x, 128, 64, w["in_bias"])   # F32 projection + bias, no BF16
    first = np.concatenate([w["special_token"][None], h]) if special else h
    assert np.array_equal(st[0], first)
    for l in range(2):
        nxt = orc.minicpm4_block(ocfg, ow.layers[l], st[l], pos=0, no_causal=1)
        assert np.array_equal(st[l + 1], nxt)
    last = orc.rms_norm(st[2][:1] if special else st[2], w["norm"], 1e-6)
    assert np.array_equal(out, last[0] if special else last)
    if special:   # the special row sees every patch row (bidirectional attention)
        x2 = x.copy()
        x2[-1] += 0.5
        assert not np.array_equal(orc.locenc_forward(ocfg, ow, x2), out)


def _lm(orc, rng, L, H, nh, nkv, hd, F, no_rope, cap):
    lws, dev = _layers(orc, rng, L, H, nh, nkv, hd, F)
    norm = (1 + rng.normal(0, 0.02, H)).astype(np.float32)
    cfg = orc.make_cfg(H, nh, nkv, hd, F, eps=1e-6, rope_theta=10000.0, no_rope=no_rope,
                       rope_ff=orc.ROPE_SHORT_FACTORS if hd == 128 else None)
    k = [np.zeros((nkv, cap, hd), np.uint16) for _ in range(L)]
    v = [np.zeros((nkv, cap, hd), np.uint16) for _ in range(L)]
    return dict(cfg=cfg, layers=lws, norm=norm, k=k, v=v, cap=cap, dev=dev)


def make_lm_update(orc, seed, with_fsq=True, L=128, E=128, Fq=64, R=128, cap=16, enc_kw=None, lm_kw=None):
    """Seeded (encoder, TSLM, RALM, projections); enc_kw / lm_kw override the block shapes
    (lm_kw: n_layers, nh, nkv, hd, F of both LMs)."""
    rng = np.random.default_rng(seed)
    enc = make_locenc(orc, seed + 1, H=E, **(enc_kw or {}))
    k = {**dict(n_layers=2, nh=4, nkv=2, hd=32, F=256), **(lm_kw or {})}
    tslm = _lm(orc, rng, k["n_layers"], L, k["nh"], k["nkv"], k["hd"], k["F"], 0, cap)
    ralm = _lm(orc, rng, k["n_layers"], R, k["nh"], k["nkv"], k["hd"], k["F"], 1, cap)

    def vec(n):
        return rng.normal(0, 0.02, n).astype(np.float32)

    pw = dict(L=L, E=E, Fq=Fq, R=R, enc_to_lm=q8(orc, rng, L, E, 0.05), enc_to_lm_bias=vec(L),
              fusion=q8(orc, rng, R, 2 * L, 0.03))
    if with_fsq:
        pw.update(fsq_in=q8(orc, rng, Fq, L, 0.1), fsq_in_bias=vec(Fq), fsq_out=q8(orc, rng, L, Fq, 0.05),
                  fsq_out_bias=vec(L))
    return enc, tslm, ralm, pw


def test_lm_update_composition(orc):
    """The chain's own structure: the TSLM and RALM caches are written at row pos only; the RALM input is
    the fusion projection of [fsq ; audio]; FSQ outputs sit on its grid before fsq_out."""
    enc, tslm, ralm, pw = make_lm_update(orc, 20)
    ecfg, ew, eow, eocfg = enc
    patch = np.random.default_rng(21).normal(0, 1, (4, 64)).astype(np.float32)
    pos = 5
    audio, base, fsq, rh = orc.lm_update(eocfg, eow, tslm, ralm, pw, patch, pos)
    for lm in (tslm, ralm):
        for k in lm["k"]:
            rows = np.nonzero(k.reshape(k.shape[0], k.shape[1], -1).any(axis=(0, 2)))[0]
            assert list(rows) == [pos]
    fe = orc.locenc_forward(eocfg, eow, patch)
    assert np.array_equal(audio, orc.linear(pw["enc_to_lm"], fe, 128, 128, pw["enc_to_lm_bias"])[0])
    h = orc.linear(pw["fsq_in"], base, 64, 128, pw["fsq_in_bias"])[0]
    q = orc.fsq_quantize(h, 9.0)
    assert np.array_equal(fsq, orc.linear(pw["fsq_out"], q, 128, 64, pw["fsq_out_bias"])[0])


def test_lm_update_without_fsq_passes_the_hidden(orc):
    enc, tslm, ralm, pw = make_lm_update(orc, 30, with_fsq=False)
    patch = np.random.default_rng(31).normal(0, 1, (4, 64)).astype(np.float32)
    audio, base, fsq, rh = orc.lm_update(enc[3], enc[2], tslm, ralm, pw, patch, 0)
    assert np.array_equal(fsq, base)


def _fresh_caches(lm):
    for k in lm["k"] + lm["v"]:
        k[...] = 0


def test_prompt_prefill_structure(orc):
    """gen_prompt_eval_range's composition: caches are written at rows [pos, pos + n) only; the RALM input
    is the fusion of [base ; 0] -- the fusion's second-half columns cannot matter, its first half must."""
    enc, tslm, ralm, pw = make_lm_update(orc, 40, with_fsq=False, cap=24)
    rng = np.random.default_rng(41)
    x = rng.normal(0, 1, (6, 128)).astype(np.float32)
    pos = 3
    base, rh = orc.prompt_prefill(tslm, ralm, pw, x, pos)
    assert base.shape == (6, 128) and rh.shape == (6, 128)
    for lm in (tslm, ralm):
        for k in lm["k"]:
            rows = np.nonzero(k.reshape(k.shape[0], k.shape[1], -1).any(axis=(0, 2)))[0] if k.ndim == 3 else \
                np.nonzero(k.reshape(2, lm["cap"], -1).any(axis=(0, 2)))[0]
            assert list(rows) == list(range(pos, pos + 6))
    # the second half of every fusion row (rows of 2L inputs) multiplies zeros
    R, L = pw["R"], pw["L"]
    rb = 2 * L // 32 * 34
    fus = pw["fusion"].reshape(R, rb).copy()
    fus[:, rb // 2:] = orc.quantize_rows(rng.normal(0, 1, (R, L)).astype(np.float32), orc.QUANT_REF).reshape(R, -1)
    pw2 = dict(pw, fusion=fus.reshape(-1))
    for lm in (tslm, ralm):
        _fresh_caches(lm)
    base2, rh2 = orc.prompt_prefill(tslm, ralm, pw2, x, pos)
    assert np.array_equal(base2, base) and np.array_equal(rh2, rh)
    # ... and the first half does
    fus3 = pw["fusion"].reshape(R, rb).copy()
    fus3[:, :rb // 2] = fus[:, rb // 2:]
    for lm in (tslm, ralm):
        _fresh_caches(lm)
    _, rh3 = orc.prompt_prefill(tslm, ralm, dict(pw, fusion=fus3.reshape(-1)), x, pos)
    assert not np.allclose(rh3, rh, atol=1e-3)


def test_prompt_prefill_in_chunks_equals_whole(orc):
    """A prompt evaluated in two ranges (gen_prompt_eval_range's pos_start) gives the same hidden states
    and caches as in one: the base LM and the RALM are causal over positions."""
    enc, tslm, ralm, pw = make_lm_update(orc, 50, with_fsq=False, cap=24)
    x = np.random.default_rng(51).normal(0, 1, (9, 128)).astype(np.float32)
    base, rh = orc.prompt_prefill(tslm, ralm, pw, x, 0)
    caches = [a.copy() for lm in (tslm, ralm) for a in lm["k"] + lm["v"]]
    for lm in (tslm, ralm):
        _fresh_caches(lm)
    b1, r1 = orc.prompt_prefill(tslm, ralm, pw, x[:4], 0)
    b2, r2 = orc.prompt_prefill(tslm, ralm, pw, x[4:], 4)
    assert np.array_equal(np.concatenate([b1, b2]), base) and np.array_equal(np.concatenate([r1, r2]), rh)
    for a, b in zip(caches, [a for lm in (tslm, ralm) for a in lm["k"] + lm["v"]]):
        assert np.array_equal(a, b)


def test_embed_rows_q8_0_closed_form(orc):
    """The Q8_0 embedding rows: each element is int8 q times the block's fp16 scale, read straight from
    the 34-byte blocks; ids outside the table read row 0."""
    rng = np.random.default_rng(60)
    rows, k = 11, 96
    table = orc.quantize_rows(rng.normal(0, 0.5, (rows, k)).astype(np.float32), orc.QUANT_REF)
    ids = np.array([3, 0, 10, -1, 11, 7, 1 << 20], np.int32)
    got = orc.embed_rows_q8_0(table, rows, k, ids)
    blocks = table.reshape(rows, k // 32, 34)
    d = blocks[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float32)
    q = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    full = (q * d[:, :, None]).reshape(rows, k)
    want = full[[3, 0, 10, 0, 0, 7, 0]]
    assert np.array_equal(got, want)
