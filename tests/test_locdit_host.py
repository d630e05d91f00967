"""CPU checks of the LocDiT / CFM host logic and of the oracle's LocDiT restatement.

The library's host helpers (sinusoid embedding, CFM schedules, zero-init step
count) must equal the oracle bit for bit; the oracle's schedules are pinned by
the reference's known answers (tests/test_oracle.py).  The LocDiT forward of
the oracle is pinned structurally: with no blocks the velocity reduces to
out_proj(RMSNorm(bf16(in_proj x + b))) of the x rows alone, so mu, t and cond
cannot leak in and the slice must start at row 3 + Pc.
"""
import numpy as np
import pytest

from locdit_case import make_inputs, make_locdit


@pytest.mark.parametrize("t", [0.0, 1.0, 0.5, 0.123456, 0.9, 1e-3])
@pytest.mark.parametrize("dim", [1024, 64, 2])
def test_host_sinusoid_matches_oracle(orc, t, dim):
    import vxm

    got = vxm.host_sinusoid_embed(t, dim)
    assert np.array_equal(got.view(np.uint32), orc.sinusoid(t, dim).view(np.uint32))


@pytest.mark.parametrize("n", [1, 2, 5, 10, 24, 100])
def test_host_cfm_schedule_matches_oracle(orc, n):
    import vxm

    for k in range(-1, n + 2):
        assert vxm.host_cfm_t(k, n, vxm.CFM_SWAY) == orc.sway_t(k, n)
        assert vxm.host_cfm_t(k, n, vxm.CFM_UNIFORM) == orc.uniform_t(k, n)
    assert vxm.host_cfm_zero_star_steps(n) == orc.zero_star_steps(n)


def _proj_bf16(orc, w, b, x, N, K):
    """bf16(ggml_mul_mat(W, x) + b) through the oracle's pinned mul_mat and BF16."""
    y = orc.mul_mat(w, orc.quantize_rows(x, orc.QUANT_X86), N, K, x.shape[0])
    return orc.bf16_round(y + (b if b is not None else 0.0))


def test_oracle_locdit_without_blocks_is_x_path_only(orc):
    H, feat, P, Pc = 64, 32, 3, 5
    cfg, w, ow, ocfg = make_locdit(orc, 1, H, 0, 2, 2, 32, 128, feat)
    x, cond, mu = make_inputs(2, P, Pc, feat, H)
    v = orc.locdit_forward(ocfg, ow, x, cond, 0.7, 0.0, mu)
    h = _proj_bf16(orc, w["in_proj"], w["in_bias"], x, H, feat)
    ref = _proj_bf16(orc, w["out_proj"], w["out_bias"], orc.rms_norm(h, w["norm"], 1e-6), feat, H)
    assert np.array_equal(v, ref)
    # nothing but x reaches the output
    v2 = orc.locdit_forward(ocfg, ow, x, cond[::-1].copy(), 0.1, 0.3, None)
    assert np.array_equal(v, v2)


def test_oracle_locdit_blocks_mix_the_sequence(orc):
    H, feat, P, Pc = 64, 32, 3, 4
    cfg, w, ow, ocfg = make_locdit(orc, 3, H, 1, 2, 2, 32, 128, feat)
    x, cond, mu = make_inputs(4, P, Pc, feat, H)
    v = orc.locdit_forward(ocfg, ow, x, cond, 0.7, 0.0, mu)
    assert not np.array_equal(v, orc.locdit_forward(ocfg, ow, x, cond, 0.7, 0.0, None))
    assert not np.array_equal(v, orc.locdit_forward(ocfg, ow, x, cond, 0.2, 0.0, mu))
    assert not np.array_equal(v, orc.locdit_forward(ocfg, ow, x, cond + 1.0, 0.7, 0.0, mu))
    assert np.array_equal(v, orc.locdit_forward(ocfg, ow, x, cond, 0.7, 0.0, mu))


def test_oracle_cfm_solve_is_the_reference_loop(orc):
    """orc_cfm_solve against the loop of src/gen_step.c:583-649 written from the
    oracle's pinned pieces (forward, schedule, CFG-Zero*, BF16)."""
    H, feat, P, Pc = 64, 32, 2, 3
    cfg, w, ow, ocfg = make_locdit(orc, 5, H, 1, 2, 2, 32, 128, feat)
    x0, cond, mu = make_inputs(6, P, Pc, feat, H)
    for sched, tfun in ((0, orc.sway_t), (1, orc.uniform_t)):
        for cfg_value, m in ((2.0, mu), (1.0, mu), (2.0, None)):
            n = 5
            got = orc.cfm_solve(ocfg, ow, x0, cond, m, n, cfg_value, sched, 1)
            x = x0.copy()
            for step in range(orc.zero_star_steps(n), n):
                t, nt = tfun(step, n), tfun(step + 1, n)
                dt = orc.bf16_round(np.float32([-(np.float32(t) - np.float32(nt))]))[0]
                vc = orc.locdit_forward(ocfg, ow, x, cond, t, 0.0, m)
                if cfg_value != 1.0 and m is not None:
                    vu = orc.locdit_forward(ocfg, ow, x, cond, t, 0.0, None)
                    _, v = orc.cfg_zero_star(vu, vc, cfg_value)
                else:
                    v = vc
                x = orc.bf16_round(x + orc.bf16_round(np.float32(dt) * v))
            assert np.array_equal(got, x), (sched, cfg_value, m is None)


@pytest.mark.parametrize("hd,use_ff", [(64, False), (128, True), (128, False), (32, False)])
def test_host_rope_table_rotates_like_oracle(orc, hd, use_ff):
    """Rotating with the library's (cos, sin) table reproduces orc_rope_neox bit for bit."""
    import vxm

    ff = orc.ROPE_SHORT_FACTORS if use_ff else None
    n_pos, nh = 700, 2
    tab = vxm.host_rope_cache(10000.0, hd, ff, 0, n_pos)
    assert np.array_equal(tab[300:320], vxm.host_rope_cache(10000.0, hd, ff, 300, 20))
    rng = np.random.default_rng(hd)
    half = hd // 2
    for pos in (0, 1, 5, 17, 255, 511, 699):
        x = orc.bf16_round(rng.normal(0, 1, nh * hd).astype(np.float32))
        ref = orc.rope_neox(x, nh, hd, pos, 10000.0, ff)
        v = x.reshape(nh, hd)
        c, s = tab[pos, :, 0], tab[pos, :, 1]
        x0, x1 = v[:, :half], v[:, half:]
        y = np.concatenate([orc.bf16_round(x0 * c - x1 * s), orc.bf16_round(x0 * s + x1 * c)], axis=1)
        assert np.array_equal(y.reshape(-1), ref), pos


def test_oracle_locdit_states_chain(orc):
    """The per-block states of the oracle: each is the block applied to the previous,
    the first holds the assembled sequence (x rows = bf16(in_proj x + b))."""
    H, feat, P, Pc = 64, 32, 3, 4
    cfg, w, ow, ocfg = make_locdit(orc, 7, H, 2, 2, 2, 32, 128, feat)
    x, cond, mu = make_inputs(8, P, Pc, feat, H)
    v, st = orc.locdit_states(ocfg, ow, x, cond, 0.3, 0.0, mu)
    assert np.array_equal(v, orc.locdit_forward(ocfg, ow, x, cond, 0.3, 0.0, mu))
    assert np.array_equal(st[0][:2], mu)
    assert np.array_equal(st[0][3 + Pc:], _proj_bf16(orc, w["in_proj"], w["in_bias"], x, H, feat))
    assert np.array_equal(st[0][3:3 + Pc], _proj_bf16(orc, w["cond_proj"], w["cond_bias"], cond, H, feat))
    for l in range(2):
        assert np.array_equal(st[l + 1], orc.minicpm4_block(ocfg, ow.layers[l], st[l], pos=0, no_causal=1))


def test_oracle_block_sensitivity_to_one_ulp(orc):
    """The measurement behind the full-width block bar of the GPU tests: moving ONE
    element of a block's input by one BF16 ulp moves the oracle's own output by a
    relative L2 of a few 1e-3 (far outside a 1e-3 per-element bar), yet within
    2^-6 of each row's scale."""
    cfg, w, ow, ocfg = make_locdit(orc, 51, 1024, 1, 16, 16, 64, 4096, 64)
    x, cond, mu = make_inputs(52, 4, 17, 64, 1024)
    _, st = orc.locdit_states(ocfg, ow, x, cond, 0.6, 0.0, mu)
    base = st[1]
    worst_rel = 0.0
    for (r, c) in ((20, 652), (12, 276), (7, 41)):
        p = st[0].copy()
        p.view(np.uint32)[r, c] += 1 << 16
        y = orc.minicpm4_block(ocfg, ow.layers[0], p, pos=0, no_causal=1).astype(np.float64)
        rel = np.linalg.norm(y - base) / np.linalg.norm(base)
        row = (np.abs(y - base) / np.abs(base).max(axis=1, keepdims=True)).max()
        worst_rel = max(worst_rel, rel)
        assert row <= 2.0 ** -6
    assert worst_rel > 1e-3


def test_oracle_velocity_sensitivity_to_one_ulp(orc):
    """The measurement behind the velocity bar of the GPU tests: the velocity of one
    full-width block (final norm of the x rows, out_proj, BF16), recomputed from the
    block's input with ONE element moved by one BF16 ulp, moves the oracle's own
    velocity by a relative L2 above the block bar's 5e-3 for most seeds and, over the
    eight seeds and six random elements each, by at most 1e-2 relative L2 and 2^-5 of
    a row's scale."""
    worst_rel = worst_row = 0.0
    above = 0
    for seed in (51, 101, 202, 303, 404, 505, 606, 707):
        cfg, w, ow, ocfg = make_locdit(orc, seed, 1024, 1, 16, 16, 64, 4096, 64)
        x, cond, mu = make_inputs(seed + 1, 4, 17, 64, 1024)
        v, st = orc.locdit_states(ocfg, ow, x, cond, 0.6, 0.0, mu)

        def vel(s0):
            seq = orc.minicpm4_block(ocfg, ow.layers[0], s0, pos=0, no_causal=1)
            hn = orc.rms_norm(seq[3 + 17:], ow.norm, 1e-6)
            return orc.bf16_round(orc.linear(ow.out_proj, hn, ow.feat, 1024, bias=ow.out_bias)).astype(np.float64)

        assert np.array_equal(vel(st[0]), v), "the composition is the oracle's velocity"
        rng = np.random.default_rng(seed)
        seed_rel = 0.0
        for _ in range(6):
            p = st[0].copy()
            p.view(np.uint32)[int(rng.integers(0, 24)), int(rng.integers(0, 1024))] += 1 << 16
            y = vel(p)
            rel = np.linalg.norm(y - v) / np.linalg.norm(v)
            row = (np.abs(y - v) / np.abs(v).max(axis=1, keepdims=True)).max()
            seed_rel, worst_row = max(seed_rel, rel), max(worst_row, row)
        worst_rel = max(worst_rel, seed_rel)
        above += seed_rel > 5e-3
    assert above >= 4 and worst_rel > 8e-3 and worst_row > 2.0 ** -6
    assert worst_rel <= 1e-2 and worst_row <= 2.0 ** -5


def test_oracle_cfm_trajectory_sensitivity(orc):
    """The measurement behind the trajectory bar of the GPU tests: one BF16 ulp on
    one element of x0 moves the oracle's own 3-step CFG trajectory (full width,
    one block) by a relative L2 above 1e-2."""
    cfg, w, ow, ocfg = make_locdit(orc, 61, 1024, 1, 16, 16, 64, 4096, 64)
    x0, cond, mu = make_inputs(62, 4, 17, 64, 1024)
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 3, 2.0, 1, 0).astype(np.float64)
    x = x0.copy()
    x.view(np.uint32)[2, 40] += 1 << 16
    y = orc.cfm_solve(ocfg, ow, x, cond, mu, 3, 2.0, 1, 0)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert 1e-2 < rel < 3e-2
