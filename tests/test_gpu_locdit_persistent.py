"""GPU parity of the single-launch LocDiT / LocEnc blocks (k_locdit_persistent) against the oracle.

The persistent kernel runs every block of an evaluation in one launch and
hands each phase's output to the next through tagged words; its rounding
steps are those of the launch-based kernels, the attention's P.V sum runs in
the oracle's order and only the fp32 order of the matrix products differs.
One full-width block meets the bars of test_gpu_locdit.py and
test_gpu_lm_update.py through the whole driver: the LocDiT velocity (16 x 64
heads) the velocity bar over eight seeds, the reference-shape solve (16 / 2 x
128) the trajectory bar, the encoder's hidden rows the block sensitivity bar.
Every block of one 12-block launch (LocDiT at both shapes, both CFG branches,
the encoder) meets the block sensitivity bar against the oracle's block fed the
launch's own input to it (read back with vxm_locdit_set_block_dump).  The
12-block outputs meet the deep-stack gross bar against the oracle (relative L2 <
5e-2), and on prefixes of 2, 4, 8 and 12 blocks stay within twice the
launch-based path's distance from the oracle (+ 1e-3) of that path.
Solves replayed from a recorded HIP graph are bit-identical to the eager solve.
"""

import numpy as np
import pytest

from locdit_case import make_inputs, make_locdit
from test_gpu_minicpm4 import assert_layer_close

pytestmark = pytest.mark.gpu

MHA = dict(H=1024, L=12, nh=16, nkv=16, hd=64, F=4096, feat=64)   # 24 rows per branch
GQA = dict(H=1024, L=12, nh=16, nkv=2, hd=128, F=4096, feat=64)   # the reference's LocDiT: 11 rows per branch
PC = {"mha": 17, "gqa": 4}


def _dev(a):
    import torch

    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _model(vxm_ctx, orc, seed, dims):
    import vxm

    cfg, w, ow, ocfg = make_locdit(orc, seed, dims["H"], dims["L"], dims["nh"], dims["nkv"], dims["hd"], dims["F"],
                                   dims["feat"], True)
    return vxm.LocDiT(vxm_ctx, cfg, w), ow, ocfg


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


@pytest.mark.parametrize("seed", [51, 101, 202, 303, 404, 505, 606, 707])
def test_persistent_locdit_one_block_full_width_mha(vxm_ctx, orc, seed):
    """One 16 x 64 block at full width through the whole driver (time MLP, projections,
    assembly, final norm, out_proj) in one persistent launch, over eight seeds: the
    velocity bar (the block bar holds only for some seeds, on both paths alike)."""
    import vxm
    from test_gpu_locdit import assert_velocity_close

    m, ow, ocfg = _model(vxm_ctx, orc, seed, dict(MHA, L=1))
    m.set_block_mode(vxm.DECODE_PERSISTENT)
    x, cond, mu = make_inputs(seed + 1, 4, 17, 64, 1024)
    print(f"persistent locdit L=1 mha seed {seed}", flush=True)
    v = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    m.check()
    assert_velocity_close(v, orc.locdit_forward(ocfg, ow, x, cond, 0.6, 0.0, mu),
                          what=f"persistent locdit L=1 mha seed {seed}")
    m.free()


def test_persistent_locdit_one_block_sway_gqa(vxm_ctx, orc):
    """The reference's solve with one 16 / 2 x 128 block: 10 sway steps, CFG 2.0, CFG-Zero*,
    both branches of 11 rows in one persistent launch per evaluation, against the oracle's
    loop (the trajectory bar of test_gpu_locdit.py)."""
    import vxm
    from test_gpu_locdit import assert_trajectory_close

    m, ow, ocfg = _model(vxm_ctx, orc, 73, dict(GQA, L=1))
    m.set_block_mode(vxm.DECODE_PERSISTENT)
    x0, cond, mu = make_inputs(74, 4, 4, 64, 1024)
    x = _dev(x0)
    print("persistent cfm L=1 gqa", flush=True)
    m.cfm_solve(x, _dev(cond), _dev(mu), 10, 2.0, vxm.CFM_SWAY, True)
    m.check()
    assert_trajectory_close(x.cpu().numpy(), orc.cfm_solve(ocfg, ow, x0, cond, mu, 10, 2.0, 0, 1),
                            what="persistent cfm L=1 gqa")
    m.free()


def _locenc(vxm_ctx, orc, seed, L, special):
    import vxm
    from test_lm_update_host import make_locenc

    cfg, w, ow, ocfg = make_locenc(orc, seed, H=1024, L=L, nh=16, nkv=2, hd=128, F=4096, special=special)
    return vxm.LocEnc(vxm_ctx, cfg, w), ow, ocfg


@pytest.mark.parametrize("special", [True, False])
def test_persistent_locenc_one_block(vxm_ctx, orc, special):
    """The encoder's hidden rows after one full-width block (5 rows with the special token,
    4 without) and the final norm, from one persistent launch: the block sensitivity bar."""
    import vxm
    from test_gpu_locdit import assert_sensitivity_close

    enc, ow, ocfg = _locenc(vxm_ctx, orc, 141, 1, special)
    enc.set_block_mode(vxm.DECODE_PERSISTENT)
    x = np.random.default_rng(142).normal(0, 1, (4, 64)).astype(np.float32)
    print(f"persistent locenc L=1 special={special}", flush=True)
    out = enc.forward(_dev(x)).cpu().numpy()
    enc.check()
    assert_sensitivity_close(out.reshape(-1, 1024), orc.locenc_forward(ocfg, ow, x).reshape(-1, 1024),
                             what="persistent locenc L=1")
    enc.free()


def test_persistent_locenc_full_size(vxm_ctx, orc):
    """The 12-block encoder (5 rows): within the deep-stack bar of the oracle, and no farther
    from the launch-based path than that path is from the oracle (plus the same bar)."""
    import vxm

    enc, ow, ocfg = _locenc(vxm_ctx, orc, 151, 12, True)
    x = np.random.default_rng(152).normal(0, 1, (4, 64)).astype(np.float32)
    ref = orc.locenc_forward(ocfg, ow, x)
    print("persistent locenc L=12", flush=True)
    enc.set_block_mode(vxm.DECODE_PERSISTENT)
    op = enc.forward(_dev(x)).cpu().numpy()
    enc.check()
    enc.set_block_mode(vxm.DECODE_KERNELS)
    ok = enc.forward(_dev(x)).cpu().numpy()
    rp, rk, rpk = _rel(op, ref), _rel(ok, ref), _rel(op, ok)
    print(f"locenc: persistent-oracle {rp:.3e}  kernels-oracle {rk:.3e}  persistent-kernels {rpk:.3e}")
    assert np.isfinite(op).all() and rp < 5e-2
    assert rpk < rk + 5e-2
    enc.free()


@pytest.mark.parametrize("shape", ["mha", "gqa"])
def test_persistent_twelve_blocks_against_oracle_and_kernels(vxm_ctx, orc, shape):
    """The 12-block velocity: within the deep-stack bar of the oracle, and no farther from
    the launch-based path than that path is from the oracle (plus the same bar)."""
    import vxm

    dims = MHA if shape == "mha" else GQA
    m, ow, ocfg = _model(vxm_ctx, orc, 111, dims)
    x, cond, mu = make_inputs(112, 4, PC[shape], 64, 1024)
    ref = orc.locdit_forward(ocfg, ow, x, cond, 0.6, 0.0, mu)
    print(f"persistent L=12 {shape}", flush=True)
    m.set_block_mode(vxm.DECODE_PERSISTENT)
    vp = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    m.check()
    m.set_block_mode(vxm.DECODE_KERNELS)
    vk = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    rp, rk, rpk = _rel(vp, ref), _rel(vk, ref), _rel(vp, vk)
    print(f"{shape}: persistent-oracle {rp:.3e}  kernels-oracle {rk:.3e}  persistent-kernels {rpk:.3e}")
    assert np.isfinite(vp).all() and rp < 5e-2
    assert rpk < rk + 5e-2
    m.free()


@pytest.mark.parametrize("shape", ["mha", "gqa"])
def test_persistent_cfm_graph_replays(vxm_ctx, orc, shape):
    """The CFM solve (both branches in one batch) on the persistent blocks: the first
    non-zero step within the deep-stack bar of the oracle's loop; ten steps eager,
    recorded and replayed (with eager forwards in between) bit-identical."""
    import torch
    import vxm

    dims = MHA if shape == "mha" else GQA
    m, ow, ocfg = _model(vxm_ctx, orc, 121, dims)
    m.set_block_mode(vxm.DECODE_PERSISTENT)
    x0, cond, mu = make_inputs(122, 4, PC[shape], 64, 1024)
    cd, md = _dev(cond), _dev(mu)
    sched = vxm.CFM_UNIFORM if shape == "mha" else vxm.CFM_SWAY
    x = _dev(x0)
    print(f"persistent cfm {shape}", flush=True)
    m.cfm_solve(x, cd, md, 2, 2.0, sched, True)
    m.check()
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 2, 2.0, sched, 1)
    rel = _rel(x.cpu().numpy(), ref)
    print(f"{shape} cfm 2 steps: rel_l2 {rel:.3e}")
    assert rel < 1e-1
    x0d = _dev(x0)
    other = _dev(x0[:1])
    outs = []
    for rep in range(4):   # eager, recorded + replayed, replayed, replayed
        x = x0d.clone()
        m.cfm_solve(x, cd, md, 10, 2.0, sched, True)
        torch.cuda.synchronize()
        outs.append(x.cpu().numpy())
        m.forward(other, None, 0.25)
        m.check()
    assert np.isfinite(outs[0]).all() and not np.array_equal(outs[0], x0)
    for rep in range(1, 4):
        assert np.array_equal(outs[rep], outs[0]), f"run {rep}"
    m.free()


def test_persistent_mode_rejects_unsupported_shape(vxm_ctx, orc):
    import vxm

    m, _, _ = _model(vxm_ctx, orc, 131, dict(H=256, L=2, nh=4, nkv=2, hd=64, F=512, feat=64))
    m.set_block_mode(vxm.DECODE_PERSISTENT)
    x = _dev(np.zeros((4, 64), np.float32))
    with pytest.raises(vxm.VxmError):
        m.forward(x, None, 0.5)
    m.set_block_mode(vxm.DECODE_AUTO)
    assert np.isfinite(m.forward(x, None, 0.5).cpu().numpy()).all()
    m.free()


def _assert_block0(d0, s0):
    d0, s0 = np.asarray(d0, np.float64), np.asarray(s0, np.float64)
    same = float((d0 == s0).mean())
    print(f"block 0 input: {same:.4f} identical")
    assert np.all(np.abs(d0 - s0) <= 2.0 ** -7 * np.abs(s0) + 1e-4) and same >= 0.99, same


def _check_blocks(orc, ocfg, layers, dump, S, what):
    """Every block of one evaluation against the oracle's block fed the evaluation's own
    input to it (segments of S rows attend within themselves), at the block sensitivity
    bar; returns the worst relative L2."""
    from test_gpu_locdit import assert_sensitivity_close

    L = len(layers)
    rows = dump.shape[1]
    worst = 0.0
    for l in range(L):
        ref = np.concatenate([orc.minicpm4_block(ocfg, layers[l], dump[l, s0:s0 + S], None, None, 0, 0, 1)
                              for s0 in range(0, rows, S)])
        assert_sensitivity_close(dump[l + 1], ref, what=f"{what} block {l}")
        worst = max(worst, _rel(dump[l + 1], ref))
    return worst


@pytest.mark.parametrize("shape", ["mha", "gqa"])
def test_persistent_every_block_of_one_launch(vxm_ctx, orc, shape):
    """Depth inside one 12-block single launch: the library writes the rows entering
    every block and the last block's output (vxm_locdit_set_block_dump); the oracle's
    block l fed the launch's own rows must give the launch's rows entering block l + 1
    at the block sensitivity bar, for blocks 1-11 too (their phases run on channel
    words, tags and tiles that block 0 never uses).  The same for the launch-based
    path."""
    import torch
    import vxm

    dims = MHA if shape == "mha" else GQA
    m, ow, ocfg = _model(vxm_ctx, orc, 161, dims)
    x, cond, mu = make_inputs(162, 4, PC[shape], 64, 1024)
    S = 3 + PC[shape] + 4
    _, states = orc.locdit_states(ocfg, ow, x, cond, 0.6, 0.0, mu)
    worst = {}
    try:
        for mode in (vxm.DECODE_PERSISTENT, vxm.DECODE_KERNELS):
            dump = torch.full((dims["L"] + 1, S, 1024), float("nan"), dtype=torch.float32, device="cuda:0")
            m.set_block_dump(dump)
            m.set_block_mode(mode)
            print(f"{shape} 12 blocks with block dump, mode {mode}", flush=True)
            m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu))
            m.check()
            m.set_block_dump(None)
            d = dump.cpu().numpy()
            assert np.isfinite(d).all(), "a block's dump was not written"
            # the rows entering block 0 (no block yet) are the oracle's up to one BF16 ulp where the
            # fp32 order of a projection moved a value across a rounding boundary
            _assert_block0(d[0], states[0])
            worst[mode] = _check_blocks(orc, ocfg, ow.layers, d, S, f"{shape} mode {mode}")
    finally:
        m.free()
    print(f"{shape}: worst block rel-L2 persistent {worst[vxm.DECODE_PERSISTENT]:.3e}, "
          f"launch by launch {worst[vxm.DECODE_KERNELS]:.3e}")


def test_persistent_every_block_of_one_cfg_launch(vxm_ctx, orc):
    """Both CFG branches (2 segments) through 12 blocks in one launch, from a one-step
    solve: every block of both segments at the block sensitivity bar."""
    import torch
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, 171, GQA)
    x0, cond, mu = make_inputs(172, 4, PC["gqa"], 64, 1024)
    S = 3 + PC["gqa"] + 4
    dump = torch.full((GQA["L"] + 1, 2 * S, 1024), float("nan"), dtype=torch.float32, device="cuda:0")
    try:
        m.set_block_mode(vxm.DECODE_PERSISTENT)
        m.set_block_dump(dump)
        print("gqa cfg solve step with block dump", flush=True)
        m.cfm_solve(_dev(x0), _dev(cond), _dev(mu), 1, 2.0, vxm.CFM_UNIFORM, False)
        m.check()
        m.set_block_dump(None)
        d = dump.cpu().numpy()
        assert np.isfinite(d).all()
        _check_blocks(orc, ocfg, ow.layers, d, S, "gqa cfg")
    finally:
        m.free()


@pytest.mark.parametrize("special", [True, False])
def test_persistent_locenc_every_block_of_one_launch(vxm_ctx, orc, special):
    """The 12-block encoder in one launch, every block against the oracle's block fed
    the launch's own rows (block sensitivity bar), and the dumped rows against the
    oracle's own states of the first block."""
    import torch
    import vxm

    enc, ow, ocfg = _locenc(vxm_ctx, orc, 181, 12, special)
    x = np.random.default_rng(182).normal(0, 1, (4, 64)).astype(np.float32)
    S = 4 + special
    _, states = orc.locenc_forward(ocfg, ow, x, states=True)
    dump = torch.full((13, S, 1024), float("nan"), dtype=torch.float32, device="cuda:0")
    try:
        enc.set_block_mode(vxm.DECODE_PERSISTENT)
        enc.set_block_dump(dump)
        print(f"locenc 12 blocks with block dump, special={special}", flush=True)
        enc.forward(_dev(x))
        enc.check()
        enc.set_block_dump(None)
        d = dump.cpu().numpy()
        assert np.isfinite(d).all()
        # the rows entering block 0 (no block yet) are the oracle's up to one BF16 ulp where the
        # fp32 order of a projection moved a value across a rounding boundary
        _assert_block0(d[0], states[0])
        _check_blocks(orc, ocfg, ow.layers, d, S, f"locenc special={special}")
    finally:
        enc.free()


@pytest.mark.parametrize("shape", ["mha", "gqa"])
def test_persistent_prefixes_track_the_launch_based_path(vxm_ctx, orc, shape):
    """The single launch on prefixes of the same 12 blocks (L = 2, 4, 8, 12): at each
    depth no farther from the launch-based path than twice that path's distance from
    the oracle plus 1e-3 (both paths share every rounding step; only the fp32 order of
    the products differs)."""
    import vxm

    dims = MHA if shape == "mha" else GQA
    cfg, w, ow, ocfg = make_locdit(orc, 191, 1024, 12, 16, dims["nkv"], dims["hd"], 4096, 64, True)
    x, cond, mu = make_inputs(192, 4, PC[shape], 64, 1024)
    for Lp in (2, 4, 8, 12):
        cp = dict(cfg, n_layers=Lp)
        wp = dict(w, layers=w["layers"][:Lp])
        owp = orc.LocDiTW(ow.layers[:Lp], ow.feat, **{n: getattr(ow, n) for n in ow.names})
        ref = orc.locdit_forward(ocfg, owp, x, cond, 0.6, 0.0, mu)
        m = vxm.LocDiT(vxm_ctx, cp, wp)
        try:
            outs = {}
            for mode in (vxm.DECODE_PERSISTENT, vxm.DECODE_KERNELS):
                m.set_block_mode(mode)
                outs[mode] = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
                m.check()
        finally:
            m.free()
        vp, vk = outs[vxm.DECODE_PERSISTENT], outs[vxm.DECODE_KERNELS]
        rp, rk, rpk = _rel(vp, ref), _rel(vk, ref), _rel(vp, vk)
        print(f"{shape} L={Lp}: persistent-oracle {rp:.3e}  kernels-oracle {rk:.3e}  persistent-kernels {rpk:.3e}")
        assert np.isfinite(vp).all() and rpk <= 2 * rk + 1e-3, (Lp, rp, rk, rpk)


@pytest.mark.parametrize("P", [8, 12])
def test_persistent_solve_x_row_limit(vxm_ctx, orc, P):
    """A CFG solve whose two branches hold 16 x rows (P = 8: the whole solve in one
    launch, out_proj on its one 16-row tile of x rows) and 24 (P = 12: beyond that
    tile, so one single launch per evaluation): on two full-width blocks the
    trajectory bar against the oracle on both block modes, and the single launches no
    farther from the launch-based path than twice that path's distance from the
    oracle plus 1e-3."""
    import vxm
    from test_gpu_locdit import assert_trajectory_close

    m, ow, ocfg = _model(vxm_ctx, orc, 211, dict(GQA, L=2))
    x0, cond, mu = make_inputs(212, P, PC["gqa"], 64, 1024)
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 3, 2.0, 1, 1)
    outs = {}
    try:
        for mode in (vxm.DECODE_PERSISTENT, vxm.DECODE_KERNELS):
            m.set_block_mode(mode)
            print(f"P={P} solve, mode {mode}", flush=True)
            x = _dev(x0)
            m.cfm_solve(x, _dev(cond), _dev(mu), 3, 2.0, vxm.CFM_UNIFORM, True)
            m.check()
            outs[mode] = x.cpu().numpy()
            assert_trajectory_close(outs[mode], ref, f"P={P} mode {mode}")
    finally:
        m.free()
    vp, vk = outs[vxm.DECODE_PERSISTENT], outs[vxm.DECODE_KERNELS]
    rk, rpk = _rel(vk, ref), _rel(vp, vk)
    print(f"P={P}: kernels-oracle {rk:.3e}  persistent-kernels {rpk:.3e}")
    assert rpk <= 2 * rk + 1e-3, (rk, rpk)
