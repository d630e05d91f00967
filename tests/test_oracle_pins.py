"""CPU pins of the oracle's LocDiT time path, CFM loop pieces and MiniCPM4 block
composition.

* Reference fixtures (tests/golden/ref_cfm.npz, packed from the reference's
  PyTorch intermediates fixtures/ref/ar000{0,1}_d00*_*.npy by
  tests/golden/pack_ref_cfm.py): the time sinusoids of every Euler step, the
  CFG-Zero* st* and blended velocity from the cond / uncond velocities, the
  Euler update from one trajectory state to the next, and the BF16 sum of the
  two time-MLP outputs.  All are weight-free relations, so the oracle must
  reproduce them bit for bit.
* The time MLP (vcpm_time_mlp_forward, src/locdit.c:140-159): with W2 = 0 the
  time row of the sequence is bf16(bf16(b2_t) + bf16(b2_dt)), checked with the
  reference's own time-MLP outputs as b2 against its t_combined; with
  permutation-identity W1 and W2 the row has a closed form in float64.
* The block composition (vcpm_minicpm4_block, src/minicpm4.c:467-532), with
  strongly different input / post-attention gains: down = 0 leaves the
  attention branch alone (block = bf16(x + attention(norm(x, g_in)))), and
  q = k = v = o = 0 leaves the MLP branch alone (block = bf16(h + mlp(norm(h,
  g_post))), h = bf16(x)).  attention() and mlp() are pinned by the
  reference's op fixtures in test_oracle.py.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

N_STEPS = 10      # the reference run's CFM steps (src/gen_step.c:583-649); step k is fixture d = k + 1
CFG_VALUE = 2.0   # its CFG scale


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(GOLDEN, "ref_cfm.npz"), allow_pickle=False)


def _v(fx, ar, d, piece):
    return fx[f"ar{ar}_d{d}_{piece}"].reshape(-1)


# ------------------------------------------------------------- reference fixtures

@pytest.mark.parametrize("ar", [0, 1])
def test_time_sinusoids_match_reference(orc, fx, ar):
    """dit_sinusoidal_t_embed (src/locdit.c:163-188) of the sway t of each evaluated
    step, and of dt = 0, equals the reference's t_sin / dt_sin for both branches."""
    import vxm

    for d in range(2, N_STEPS + 1):
        t = orc.sway_t(d - 1, N_STEPS)
        emb = orc.sinusoid(t, 1024)
        assert np.array_equal(emb, _v(fx, ar, d, "locdit_cond_t_sin")), d
        assert np.array_equal(emb, _v(fx, ar, d, "locdit_uncond_t_sin")), d
        assert np.array_equal(vxm.host_sinusoid_embed(t, 1024), emb), d
        assert np.array_equal(orc.sinusoid(0.0, 1024), _v(fx, ar, d, "locdit_cond_dt_sin")), d


@pytest.mark.parametrize("ar", [0, 1])
def test_cfg_zero_star_matches_reference(orc, fx, ar):
    """vcpm_cfm_cfg_zero_star (src/cfm_solver.c:65-93) on the reference's cond /
    uncond velocities gives its st* and blended velocity bit for bit."""
    for d in range(2, N_STEPS + 1):
        st, blend = orc.cfg_zero_star(_v(fx, ar, d, "cfm_velocity_uncond"), _v(fx, ar, d, "cfm_velocity_cond"),
                                      CFG_VALUE)
        assert np.float32(st) == _v(fx, ar, d, "cfm_cfg_st_star")[0], d
        assert np.array_equal(blend, _v(fx, ar, d, "cfm_velocity_blend")), d


@pytest.mark.parametrize("ar", [0, 1])
def test_euler_trajectory_matches_reference(orc, fx, ar):
    """The CFM loop's schedule and update: the first step is the zero-init step
    (skipped, zero velocity), then x_{k+1} = bf16(x_k + bf16(dt_k * v_k)) with
    dt_k from the sway schedule reproduces every trajectory state, and the
    final state is the reference's CFM output."""
    assert orc.zero_star_steps(N_STEPS) == 1
    x = fx[f"ar{ar}_cfm_noise"].reshape(-1)
    assert np.array_equal(x, _v(fx, ar, 0, "cfm_traj_state"))
    assert not _v(fx, ar, 1, "cfm_velocity_blend").any()
    assert np.array_equal(_v(fx, ar, 1, "cfm_traj_state"), x)
    for d in range(2, N_STEPS + 1):
        x = orc.cfm_euler_update(x, _v(fx, ar, d, "cfm_velocity_blend"), orc.cfm_step_dt(d - 1, N_STEPS, 0))
        assert np.array_equal(x, _v(fx, ar, d, "cfm_traj_state")), d
    assert np.array_equal(x, fx[f"ar{ar}_cfm_clean"].reshape(-1))
    # a plausible slip: dt of the uniform grid instead of the sway schedule
    y = orc.cfm_euler_update(_v(fx, ar, 2, "cfm_traj_state"), _v(fx, ar, 3, "cfm_velocity_blend"),
                             orc.cfm_step_dt(2, N_STEPS, 1))
    assert not np.array_equal(y, _v(fx, ar, 3, "cfm_traj_state"))


# ------------------------------------------------------------- the time MLP

def _zero_q8(orc, n, k):
    return orc.quantize_rows(np.zeros((n, k), np.float32), orc.QUANT_REF)


def _perm_identity_q8(orc, perm, k, value=1.0):
    """Q8_0 rows with one nonzero per row: row i holds `value` at column perm[i]."""
    w = np.zeros((len(perm), k), np.float32)
    w[np.arange(len(perm)), perm] = value
    return orc.quantize_rows(w, orc.QUANT_REF)


def _time_locdit(orc, H, feat, t_w1, t_w2, dt_w1, dt_w2, t_b1, t_b2, dt_b1, dt_b2):
    """A LocDiT with no blocks (only the sequence assembly and the time MLPs matter)."""
    rng = np.random.default_rng(H)
    q = orc.quantize_rows(rng.normal(0, 0.05, (H, feat)).astype(np.float32), orc.QUANT_REF)
    qo = orc.quantize_rows(rng.normal(0, 0.05, (feat, H)).astype(np.float32), orc.QUANT_REF)
    w = orc.LocDiTW([], feat, in_proj=q, cond_proj=q, out_proj=qo, norm=np.ones(H, np.float32),
                    t_w1=t_w1, t_w2=t_w2, dt_w1=dt_w1, dt_w2=dt_w2, t_b1=t_b1, t_b2=t_b2, dt_b1=dt_b1,
                    dt_b2=dt_b2)
    cfg = orc.make_cfg(H, 8, 8, H // 8, 4 * H)
    return cfg, w


@pytest.mark.parametrize("ar,d", [(0, 2), (0, 7), (1, 10)])
def test_time_row_with_zero_w2_is_the_reference_combine(orc, fx, ar, d):
    """W2 = 0 reduces each time MLP to bf16(b2): with the reference's time-MLP
    outputs as b2, row 2 of the sequence must be the reference's t_combined."""
    H, feat = 1024, 64
    rng = np.random.default_rng(d)
    tf, dtf = _v(fx, ar, d, "locdit_cond_t_feat"), _v(fx, ar, d, "locdit_cond_dt_feat")
    w1 = orc.quantize_rows(rng.normal(0, 0.03, (H, H)).astype(np.float32), orc.QUANT_REF)
    b1 = rng.normal(0, 0.5, H).astype(np.float32)
    cfg, w = _time_locdit(orc, H, feat, w1, _zero_q8(orc, H, H), w1, _zero_q8(orc, H, H), b1, tf, b1, dtf)
    x = rng.normal(0, 1, (2, feat)).astype(np.float32)
    _, st = orc.locdit_states(cfg, w, x, x, orc.sway_t(d - 1, N_STEPS), 0.0, None)
    assert np.array_equal(st[0][2], _v(fx, ar, d, "locdit_cond_t_combined"))
    # b1 in place of b2 (a swapped bias) does not give it
    cfg2, w2 = _time_locdit(orc, H, feat, w1, _zero_q8(orc, H, H), w1, _zero_q8(orc, H, H), tf, b1, dtf, b1)
    _, st2 = orc.locdit_states(cfg2, w2, x, x, orc.sway_t(d - 1, N_STEPS), 0.0, None)
    assert not np.array_equal(st2[0][2], st[0][2])


def _f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def _perm_linear_closed_form(orc, x, perm, b, value):
    """ggml_mul_mat(W, x) + b, BF16, for W with the single entry `value` at column
    perm[i] of row i: the only nonzero block term of row i is (127 qx[perm[i]]) *
    (d_w d_x), the fp32 rounding of a product that float64 holds exactly (the
    integer and the fp16 x fp16 scale product are exact), and adding the other
    blocks' zero terms leaves it unchanged."""
    H = x.shape[-1]
    qs, dx = orc.split_q8(orc.quantize_rows(x[None], orc.QUANT_X86), 1, H)
    qw, dw = orc.split_q8(_perm_identity_q8(orc, perm, H, value), len(perm), H)
    q = int(qw[0][perm[0]])                           # every row quantizes alike
    dwi = dw[np.arange(len(perm)), perm // 32]        # the scale of row i's nonzero block
    term = (np.float64(q) * qs[0][perm].astype(np.float64) *
            (_f16(dwi).astype(np.float64) * _f16(dx[0][perm // 32]).astype(np.float64)))
    return orc.bf16_round((term.astype(np.float32) + b).astype(np.float32))


def _silu_bf16(h):
    s = h.astype(np.float64) / (1.0 + np.exp(-h.astype(np.float64)))
    return np.array([np.float32(v) for v in s], np.float32)


def test_time_mlp_closed_form_with_permutation_weights(orc):
    """Permutation-identity W1 / W2 (different for t and dt, and W1 != W2) make
    each time MLP bf16(P2 bf16(silu(bf16(P1 emb + b1))) + b2) with a closed form;
    row 2 = bf16(t_feat + dt_feat) must match it (silu in float64: the oracle's
    expf may move an element by one BF16 ulp at a rounding boundary)."""
    H, feat = 256, 32
    rng = np.random.default_rng(11)
    pt1, pt2, pd1, pd2 = (rng.permutation(H) for _ in range(4))
    vt, vd = 1.0, 0.5
    b = [rng.normal(0, 0.3, H).astype(np.float32) for _ in range(4)]
    cfg, w = _time_locdit(orc, H, feat, _perm_identity_q8(orc, pt1, H, vt), _perm_identity_q8(orc, pt2, H, vt),
                          _perm_identity_q8(orc, pd1, H, vd), _perm_identity_q8(orc, pd2, H, vd), *b)
    t, dt = 0.7109375, 0.25
    x = rng.normal(0, 1, (2, feat)).astype(np.float32)
    _, st = orc.locdit_states(cfg, w, x, x, t, dt, None)

    def mlp(emb, p1, p2, b1, b2, v):
        h = _perm_linear_closed_form(orc, emb, p1, b1, v)
        s = orc.bf16_round(_silu_bf16(h))
        return _perm_linear_closed_form(orc, s, p2, b2, v)

    tf = mlp(orc.sinusoid(t, H), pt1, pt2, b[0], b[1], vt)
    dtf = mlp(orc.sinusoid(dt, H), pd1, pd2, b[2], b[3], vd)
    want = orc.bf16_round((tf + dtf).astype(np.float32))
    got = st[0][2]
    ulp = np.abs(want) * 2.0 ** -8 + 1e-30
    assert np.all(np.abs(got - want) <= ulp * 1.01)
    assert (got == want).mean() >= 0.99
    # t and dt weights exchanged, or W1 and W2 exchanged: far from it
    for bad in (mlp(orc.sinusoid(t, H), pd1, pd2, b[0], b[1], vt),
                mlp(orc.sinusoid(t, H), pt2, pt1, b[0], b[1], vt)):
        wrong = orc.bf16_round((bad + dtf).astype(np.float32))
        assert (got == wrong).mean() < 0.5


# ------------------------------------------------------------- block composition

def _gains(rng, H, scale):
    return (scale * (1 + rng.normal(0, 0.3, H))).astype(np.float32)


def _layer(orc, rng, H, nh, nkv, hd, F, zero=()):
    def q8(name, n, k):
        if name in zero:
            return _zero_q8(orc, n, k)
        return orc.quantize_rows(rng.normal(0, 0.05, (n, k)).astype(np.float32), orc.QUANT_REF)

    return orc.LayerW(wq=q8("q", nh * hd, H), wk=q8("k", nkv * hd, H), wv=q8("v", nkv * hd, H),
                      wo=q8("o", H, nh * hd), wg=q8("g", F, H), wu=q8("u", F, H), wd=q8("d", H, F),
                      g_in=_gains(rng, H, 1.0), g_post=_gains(rng, H, 3.0))


@pytest.mark.parametrize("causal", [1, 0])
def test_block_with_zero_down_is_the_attention_branch(orc, causal):
    """down = 0: the MLP adds an exact zero, so the block is the attention
    residual bf16(x + attention(rms_norm(x, g_in))) -- with g_in, not g_post."""
    rng = np.random.default_rng(31 + causal)
    H, nh, nkv, hd, F, M, cap = 128, 4, 2, 32, 256, 5, 16
    lw = _layer(orc, rng, H, nh, nkv, hd, F, zero=("d",))
    cfg = orc.make_cfg(H, nh, nkv, hd, F)
    x = rng.normal(0, 1, (M, H)).astype(np.float32)
    kw = dict(k_cache=np.zeros(nkv * cap * hd, np.uint16), v_cache=np.zeros(nkv * cap * hd, np.uint16),
              capacity=cap, pos=0, no_causal=1 - causal)
    kw2 = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in kw.items()}
    y = orc.minicpm4_block(cfg, lw, x, **kw)
    att = orc.attention(cfg, lw, orc.rms_norm(x, lw.g_in, cfg.eps), **kw2)
    assert np.array_equal(y, orc.bf16_round((x + att).astype(np.float32)))
    att_post = orc.attention(cfg, lw, orc.rms_norm(x, lw.g_post, cfg.eps), **{
        k: (np.zeros_like(v) if isinstance(v, np.ndarray) else v) for k, v in kw.items()})
    assert not np.array_equal(y, orc.bf16_round((x + att_post).astype(np.float32)))


@pytest.mark.parametrize("causal", [1, 0])
def test_block_with_zero_attention_is_the_mlp_branch(orc, causal):
    """q = k = v = o = 0: attention adds an exact zero, so h = bf16(x) and the
    block is bf16(h + mlp(rms_norm(h, g_post))) -- the BF16 round of the first
    residual and g_post both matter."""
    rng = np.random.default_rng(41 + causal)
    H, nh, nkv, hd, F, M, cap = 128, 4, 2, 32, 256, 5, 16
    lw = _layer(orc, rng, H, nh, nkv, hd, F, zero=("q", "k", "v", "o"))
    cfg = orc.make_cfg(H, nh, nkv, hd, F)
    x = rng.normal(0, 1, (M, H)).astype(np.float32)   # not BF16-valued
    y = orc.minicpm4_block(cfg, lw, x, np.zeros(nkv * cap * hd, np.uint16), np.zeros(nkv * cap * hd, np.uint16),
                           cap, 0, 1 - causal)
    h = orc.bf16_round(x)
    want = orc.bf16_round((h + orc.mlp(cfg, lw, orc.rms_norm(h, lw.g_post, cfg.eps))).astype(np.float32))
    assert np.array_equal(y, want)
    # without the BF16 round of h, or with g_in in the MLP's norm: different
    skip = orc.bf16_round((x + orc.mlp(cfg, lw, orc.rms_norm(x, lw.g_post, cfg.eps))).astype(np.float32))
    swap = orc.bf16_round((h + orc.mlp(cfg, lw, orc.rms_norm(h, lw.g_in, cfg.eps))).astype(np.float32))
    assert not np.array_equal(y, skip) and not np.array_equal(y, swap)
