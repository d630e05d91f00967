"""GPU parity of the LocDiT velocity network and the device CFM loop against the oracle.

Velocities pass through BF16 after every op (src/locdit.c:118-121).  At the
small test shapes their bar is the block bar: >= 99.5% of elements within 1e-3
rel / 1e-4 abs of the oracle, every element within 4 BF16 ulps (+1e-4),
relative L2 < 1e-3.  At full width that bar holds only for some inputs, on the
launch-by-launch and single-launch paths alike (they are bit-identical to each
other there), so full-width velocities take the velocity bar (assert_velocity_close,
from the oracle's own one-ulp sensitivity of the velocity), over eight seeds.

Full-width blocks are compared one by one (each device block fed the
oracle's input to that block) against the block's intrinsic sensitivity:
Q8_0 re-quantization of every activation plus non-causal attention make one
last-bit difference anywhere (the GPU sums in a different order) spread over
the whole sequence.  The oracle's own block output moves by a relative L2 up
to ~4e-3 and up to 2^-7 of a row's scale when ONE input element moves by one
BF16 ulp (test_locdit_host.py::test_oracle_block_sensitivity_to_one_ulp).
Sensitivity bar: relative L2 < 5e-3 and every element within 2^-6 of its
row's largest magnitude.  Over 12 blocks this compounds, so the end-to-end
velocity of the deep stack carries a gross-error bar (relative L2 < 5e-2).

The loop mechanics (batching both CFG branches, CFG-Zero*, the Euler update)
are checked exactly: with every projection on the MFMA GEMM the batched solve
equals single-branch device forwards followed by the reference's host loop.
Whole trajectories against the oracle carry a wider bar: every Euler step
feeds x back through in_proj and Q8_0 re-quantization, and CFG-Zero*'s scale
st* is one BF16 scalar, so a last-bit difference anywhere moves the whole
trajectory.  The oracle's own 3-step trajectory moves by a relative L2 up to
~1.4e-2 (max 0.08) when ONE element of x0 moves by one BF16 ulp
(test_locdit_host.py::test_oracle_cfm_trajectory_sensitivity).  Trajectory
bar: relative L2 < 3e-2 and every element within 1/8 absolute.
"""
import numpy as np
import pytest

from locdit_case import make_inputs, make_locdit
from test_gpu_minicpm4 import assert_layer_close

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


SMALL = dict(H=256, L=2, nh=4, nkv=2, hd=64, F=512, feat=64)


def _model(vxm_ctx, orc, seed, H, L, nh, nkv, hd, F, feat, bias=True, keep=None):
    import vxm

    cfg, w, ow, ocfg = make_locdit(orc, seed, H, L, nh, nkv, hd, F, feat, bias)
    if keep is not None:
        keep.update(cfg=cfg, w=w)
    return vxm.LocDiT(vxm_ctx, cfg, w), ow, ocfg


@pytest.mark.parametrize("with_mu", [True, False])
@pytest.mark.parametrize("P,Pc,t,dt", [(4, 5, 0.7, 0.0), (2, 2, 1.0, 0.25), (1, 0, 0.05, 0.0)])
def test_locdit_forward_small(vxm_ctx, orc, with_mu, P, Pc, t, dt):
    m, ow, ocfg = _model(vxm_ctx, orc, 11, **SMALL)
    x, cond, mu = make_inputs(12 + P, P, Pc, SMALL["feat"], SMALL["H"])
    mu = mu if with_mu else None
    v = m.forward(_dev(x), _dev(cond) if Pc else None, t, dt, _dev(mu)).cpu().numpy()
    ref = orc.locdit_forward(ocfg, ow, x, cond, t, dt, mu)
    assert_layer_close(v, ref, what=f"locdit P={P} Pc={Pc} mu={with_mu}")
    m.free()


def test_locdit_forward_head_dim_128_no_bias(vxm_ctx, orc):
    """head_dim 128 takes the LongRoPE factors (src/minicpm4.c:183-190); biases absent."""
    m, ow, ocfg = _model(vxm_ctx, orc, 21, H=256, L=2, nh=2, nkv=1, hd=128, F=512, feat=32, bias=False)
    x, cond, mu = make_inputs(22, 3, 4, 32, 256)
    v = m.forward(_dev(x), _dev(cond), 0.4, 0.0, _dev(mu)).cpu().numpy()
    assert_layer_close(v, orc.locdit_forward(ocfg, ow, x, cond, 0.4, 0.0, mu), what="locdit hd128")
    m.free()


@pytest.mark.parametrize("schedule", [0, 1])
@pytest.mark.parametrize("cfg_value,with_mu", [(2.0, True), (1.0, True), (2.0, False)])
def test_cfm_solve_small(vxm_ctx, orc, schedule, cfg_value, with_mu):
    """The whole Euler loop on the device (both CFG branches in one batch) against
    orc_cfm_solve (two separate forwards per step)."""
    m, ow, ocfg = _model(vxm_ctx, orc, 31, **SMALL)
    x0, cond, mu = make_inputs(32, 4, 5, SMALL["feat"], SMALL["H"])
    mu = mu if with_mu else None
    x = _dev(x0)
    m.cfm_solve(x, _dev(cond), _dev(mu), 6, cfg_value, schedule, True)
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 6, cfg_value, schedule, 1)
    assert_trajectory_close(x.cpu().numpy(), ref, what=f"cfm sched={schedule} cfg={cfg_value} mu={with_mu}")
    m.free()


def assert_sensitivity_close(y, ref, what=""):
    y, ref = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    scale = np.abs(ref).max(axis=-1, keepdims=True)
    worst = (np.abs(y - ref) / np.maximum(scale, 1e-30)).max()
    print(f"{what}: rel_l2 {rel:.2e} worst/row-scale {worst:.2e}")
    assert rel < 5e-3 and worst <= 2.0 ** -6, (what, rel, worst)


def assert_velocity_close(y, ref, what=""):
    """The velocity of one full-width block (out_proj of the normed x rows, 4 x 64
    values): one BF16 flip inside the block moves the oracle's own velocity by a
    relative L2 up to 8.3e-3 and up to 1.7e-2 of a row's scale over the seeds used
    here (test_locdit_host.py::test_oracle_velocity_sensitivity_to_one_ulp), beyond
    the block bar.  Velocity bar: relative L2 < 2e-2, every element within 2^-5 of
    its row's scale."""
    y, ref = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    scale = np.abs(ref).max(axis=-1, keepdims=True)
    worst = (np.abs(y - ref) / np.maximum(scale, 1e-30)).max()
    print(f"{what}: rel_l2 {rel:.2e} worst/row-scale {worst:.2e}")
    assert rel < 2e-2 and worst <= 2.0 ** -5, (what, rel, worst)


def assert_trajectory_close(y, ref, what=""):
    y, ref = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    rel = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = np.abs(y - ref).max()
    print(f"{what}: rel_l2 {rel:.2e} max_abs {mx:.3e}")
    assert rel < 3e-2 and mx <= 1.0 / 8, (what, rel, mx)


def test_cfm_solve_matches_stepwise_forwards(vxm_ctx, orc):
    """Batched CFG steps == two single-branch forwards per step + the reference's host
    CFG-Zero* and Euler update, bit for bit (no zero-init step).  Every projection
    takes the MFMA GEMM, whose per-row result does not depend on the row count."""
    import torch
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, 41, **SMALL)
    vxm_ctx.set_path(vxm.PATH_MFMA)
    x0, cond, mu = make_inputs(42, 4, 5, SMALL["feat"], SMALL["H"])
    xd, cd, md = _dev(x0), _dev(cond), _dev(mu)
    n = 3
    x = xd.clone()
    m.cfm_solve(x, cd, md, n, 2.0, 1, False)
    xs = x0.copy()
    for step in range(n):
        t, nt = orc.uniform_t(step, n), orc.uniform_t(step + 1, n)
        dt = orc.bf16_round(np.float32([-(np.float32(t) - np.float32(nt))]))[0]
        vc = m.forward(_dev(xs), cd, t, 0.0, md).cpu().numpy()
        vu = m.forward(_dev(xs), cd, t, 0.0, None).cpu().numpy()
        _, v = orc.cfg_zero_star(vu, vc, 2.0)
        xs = orc.bf16_round(xs + orc.bf16_round(np.float32(dt) * v))
    torch.cuda.synchronize()
    vxm_ctx.set_path(vxm.PATH_AUTO)
    got = x.cpu().numpy()
    assert np.array_equal(got, xs), f"max diff {np.abs(got - xs).max()}"
    m.free()


FULL = dict(H=1024, L=12, nh=16, nkv=16, hd=64, F=4096, feat=64)


# The block bar holds only for some inputs: over other seeds the velocity of one
# full-width block misses it (at seed 101: 71.5% of elements within tolerance, 88
# BF16 ulps worst, relative L2 2.9e-3), with the launch-by-launch and single-launch
# outputs bit-identical to each other -- the fp32 order of the products against the
# oracle's, amplified by the block's sensitivity, not a kernel bug.  So full-width
# velocities take the velocity bar, over eight seeds.
SEEDS = [51, 101, 202, 303, 404, 505, 606, 707]


@pytest.mark.parametrize("seed", SEEDS)
def test_locdit_full_width_one_block(vxm_ctx, orc, seed):
    """Full width (hidden 1024, 16 x 64 heads, FFN 4096, 24 rows) with one block: the
    whole driver (time MLPs, projections, assembly, slice, norm, out_proj), launch by
    launch, at the sensitivity bar."""
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, seed, **dict(FULL, L=1))
    m.set_block_mode(vxm.DECODE_KERNELS)
    x, cond, mu = make_inputs(seed + 1, 4, 17, 64, 1024)
    print(f"locdit full width L=1 seed {seed}", flush=True)
    v = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    assert_velocity_close(v, orc.locdit_forward(ocfg, ow, x, cond, 0.6, 0.0, mu),
                          what=f"locdit full width L=1 seed {seed}")
    m.free()


@pytest.mark.parametrize("seed", SEEDS[::2])
@pytest.mark.parametrize("path", ["auto", "tiled", "gemv"])
def test_locdit_full_width_one_block_every_matmul_path(vxm_ctx, orc, path, seed):
    """The same block through each matmul path: the small-M kernel with SwiGLU fused into
    gate/up and K-split slices (AUTO at 24 rows), the tiled GEMM with the per-op SwiGLU,
    and the weight-streaming GEMV; each meets the sensitivity bar on its own."""
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, seed + 2, **dict(FULL, L=1))
    m.set_block_mode(vxm.DECODE_KERNELS)
    x, cond, mu = make_inputs(seed + 3, 4, 17, 64, 1024)
    ref = orc.locdit_forward(ocfg, ow, x, cond, 0.3, 0.0, mu)
    code = {"auto": vxm.PATH_AUTO, "tiled": vxm.PATH_MFMA_TILED, "gemv": vxm.PATH_GEMV}[path]
    try:
        vxm_ctx.set_path(code)
        v = m.forward(_dev(x), _dev(cond), 0.3, 0.0, _dev(mu)).cpu().numpy()
    finally:
        vxm_ctx.set_path(vxm.PATH_AUTO)
    assert_velocity_close(v, ref, what=f"locdit full width L=1, {path} path, seed {seed}")
    m.free()


def test_locdit_full_size_forward(vxm_ctx, orc):
    """The CFM velocity workload: hidden 1024, 12 layers, 16 x 64 heads, FFN 4096;
    4 latent tokens + 17 cond tokens + mu(2) + t(1) = 24 rows per branch.  Every
    block meets the block bar against the oracle's input to it; the end-to-end
    velocity meets the gross bar."""
    import vxm

    keep = {}
    m, ow, ocfg = _model(vxm_ctx, orc, 51, **FULL, keep=keep)
    x, cond, mu = make_inputs(52, 4, 17, 64, 1024)
    v = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    ref, states = orc.locdit_states(ocfg, ow, x, cond, 0.6, 0.0, mu)
    c = keep["cfg"]
    blocks = vxm.MiniCPM4(vxm_ctx, dict(hidden_size=c["hidden_size"], n_layers=c["n_layers"],
                                        n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"], head_dim=c["head_dim"],
                                        intermediate_size=c["intermediate_size"], rms_norm_eps=1e-6,
                                        rope_theta=10000), keep["w"]["layers"])
    for l in range(c["n_layers"]):
        h = _dev(states[l])
        blocks.block(None, l, h, 0, 1)
        assert_sensitivity_close(h.cpu().numpy(), states[l + 1], what=f"locdit block {l}")
    blocks.free()
    rel = np.linalg.norm(v.astype(np.float64) - ref) / np.linalg.norm(ref)
    print(f"end-to-end velocity rel_l2 {rel:.3e}")
    assert np.isfinite(v).all() and rel < 5e-2
    m.free()


def test_cfm_full_width_one_block(vxm_ctx, orc):
    """Full-width CFG solve (one block) over 3 uniform steps against the oracle."""
    m, ow, ocfg = _model(vxm_ctx, orc, 61, **dict(FULL, L=1))
    x0, cond, mu = make_inputs(62, 4, 17, 64, 1024)
    x = _dev(x0)
    m.cfm_solve(x, _dev(cond), _dev(mu), 3, 2.0, 1, False)
    assert_trajectory_close(x.cpu().numpy(), orc.cfm_solve(ocfg, ow, x0, cond, mu, 3, 2.0, 1, 0),
                            what="cfm full width L=1")
    m.free()


def test_cfm_full_size_one_step_and_repeatable(vxm_ctx, orc):
    """The 12-block solve: one full Euler step (t 1 -> 0, so x moves by the whole
    blended velocity, CFG 2 doubling velocity differences) within the gross bar
    of the deep stack, and ten steps finite and bit-identical across runs."""
    import torch

    m, ow, ocfg = _model(vxm_ctx, orc, 61, **FULL)
    x0, cond, mu = make_inputs(62, 4, 17, 64, 1024)
    cd, md = _dev(cond), _dev(mu)
    x = _dev(x0)
    m.cfm_solve(x, cd, md, 1, 2.0, 1, True)
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 1, 2.0, 1, 1)
    rel = np.linalg.norm(x.cpu().numpy().astype(np.float64) - ref) / np.linalg.norm(ref)
    print(f"cfm 12 blocks, 1 step: rel_l2 {rel:.3e}")
    assert rel < 1e-1
    # ten uniform steps twice: finite and bit-identical
    outs = []
    for _ in range(2):
        x = _dev(x0)
        m.cfm_solve(x, cd, md, 10, 2.0, 1, True)
        torch.cuda.synchronize()
        outs.append(x.cpu().numpy())
    assert np.isfinite(outs[0]).all() and np.array_equal(outs[0], outs[1])
    assert not np.array_equal(outs[0], x0)
    m.free()


# Widths off the small-M kernel's layout (N % 64, K % 256) and a head size off the fused
# local attention: the tiled GEMM (down: a K split outside the Euler loop) and the
# per-op attention run inside the recorded loop.
ODD = dict(H=160, L=2, nh=5, nkv=5, hd=32, F=2080, feat=64)


@pytest.mark.parametrize("cfg", ["full", "odd"])
def test_cfm_graph_replays_match_eager(vxm_ctx, orc, cfg):
    """vxm_cfm_solve records its Euler loop as a HIP graph on the second call with the
    same arguments and buffers and replays it afterwards: every replay, with eager work
    and synchronizations in between, is bit-identical to the eager first call; a call
    with other arguments runs eagerly and the recorded loop still replays correctly."""
    import torch

    dims = FULL if cfg == "full" else ODD
    m, _, _ = _model(vxm_ctx, orc, 81, **dims)
    x0, cond, mu = make_inputs(82, 4, 17, 64, dims["H"])
    cd, md = _dev(cond), _dev(mu)
    x0d = _dev(x0)
    x = torch.empty_like(x0d)
    other = _dev(x0[:1])

    def solve(n_steps=10):
        x.copy_(x0d)
        m.cfm_solve(x, cd, md, n_steps, 2.0, 1, True)
        torch.cuda.synchronize()
        return x.cpu().numpy()

    eager = solve()                      # first call with this key: eager
    assert np.isfinite(eager).all() and not np.array_equal(eager, x0)
    for rep in range(4):                 # recorded, then replayed
        assert np.array_equal(solve(), eager), f"run {rep + 2}"
        m.forward(other, None, 0.25)     # eager work on the same model between replays
        torch.cuda.synchronize()
    five = solve(5)                      # another key: eager
    assert not np.array_equal(five, eager)
    for rep in range(3):                 # back to the first key: eager, recorded, replayed
        assert np.array_equal(solve(), eager), f"return run {rep}"
    # the time rows are kept between solves of one schedule; the sway schedule has as many
    # steps (the same buffers) with other t, so its rows replace them, and back again
    x.copy_(x0d)
    m.cfm_solve(x, cd, md, 10, 2.0, 0, True)
    torch.cuda.synchronize()
    sway = x.cpu().numpy()
    assert not np.array_equal(sway, eager)
    assert np.array_equal(solve(), eager), "uniform after sway"
    x.copy_(x0d)
    m.cfm_solve(x, cd, md, 10, 2.0, 0, True)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), sway), "sway after uniform"
    # the quantizer is part of what the time rows depend on: after a switch they are formed
    # anew, as a model that only ever ran with the other quantizer forms them
    vxm_ctx.set_quant_variant(0)
    try:
        ref_q = solve()
        fresh, _, _ = _model(vxm_ctx, orc, 81, **dims)
        x.copy_(x0d)
        fresh.cfm_solve(x, cd, md, 10, 2.0, 1, True)
        torch.cuda.synchronize()
        assert np.array_equal(x.cpu().numpy(), ref_q), "time rows after a quantizer switch"
        fresh.free()
    finally:
        vxm_ctx.set_quant_variant(1)
    m.free()


def test_locdit_rejects_bad_sizes(vxm_ctx, orc):
    import vxm

    m, _, _ = _model(vxm_ctx, orc, 71, **SMALL)
    x = _dev(np.zeros((65, 64), np.float32))
    with pytest.raises(vxm.VxmError) as e:
        m.forward(x, None, 0.5)          # P * feat = 4160 > 2048
    assert e.value.code == 1
    with pytest.raises(vxm.VxmError):
        m.cfm_solve(_dev(np.zeros((2, 64), np.float32)), None, None, 4, 2.0, 7, True)
    m.free()


# The reference's own LocDiT (src/gen_init.c:280-283,424-441; src/gen_step.c:442-649): hidden 1024,
# 12 layers, 16 query heads and 2 KV heads of 128 (LongRoPE short factors), FFN 4 x hidden; per CFG
# branch mu (2 rows) + t (1) + the previous patch as cond (4) + the latent patch (4) = 11 rows; 10 sway
# steps with CFG-Zero* at CFG 2.0.
REF = dict(H=1024, L=12, nh=16, nkv=2, hd=128, F=4096, feat=64)


def test_locdit_reference_shape_forward(vxm_ctx, orc):
    """Every block of the reference-shape LocDiT (GQA 16 / 2 x 128, 11 rows per branch) meets the block
    sensitivity bar against the oracle's input to it; the velocity meets the gross bar."""
    import vxm

    keep = {}
    m, ow, ocfg = _model(vxm_ctx, orc, 71, **REF, keep=keep)
    x, cond, mu = make_inputs(72, 4, 4, 64, 1024)
    v = m.forward(_dev(x), _dev(cond), 0.6, 0.0, _dev(mu)).cpu().numpy()
    ref, states = orc.locdit_states(ocfg, ow, x, cond, 0.6, 0.0, mu)
    assert states[0].shape[0] == 11
    c = keep["cfg"]
    blocks = vxm.MiniCPM4(vxm_ctx, dict(hidden_size=1024, n_layers=12, n_heads=16, n_kv_heads=2, head_dim=128,
                                        intermediate_size=4096, rms_norm_eps=1e-6, rope_theta=10000),
                          keep["w"]["layers"])
    for l in range(c["n_layers"]):
        h = _dev(states[l])
        blocks.block(None, l, h, 0, 1)
        assert_sensitivity_close(h.cpu().numpy(), states[l + 1], what=f"reference locdit block {l}")
    blocks.free()
    rel = np.linalg.norm(v.astype(np.float64) - ref) / np.linalg.norm(ref)
    print(f"reference-shape velocity rel_l2 {rel:.3e}")
    assert np.isfinite(v).all() and rel < 5e-2
    m.free()


@pytest.mark.parametrize("path", ["auto", "tiled"])
def test_cfm_reference_shape_one_block_sway(vxm_ctx, orc, path):
    """The reference's solve at full width with one block: 10 sway steps, CFG 2.0, CFG-Zero* (its zero
    first step), both branches of 11 rows in one batch, against the oracle's loop."""
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, 73, **dict(REF, L=1))
    x0, cond, mu = make_inputs(74, 4, 4, 64, 1024)
    x = _dev(x0)
    code = {"auto": vxm.PATH_AUTO, "tiled": vxm.PATH_MFMA_TILED}[path]
    try:
        vxm_ctx.set_path(code)
        m.cfm_solve(x, _dev(cond), _dev(mu), 10, 2.0, vxm.CFM_SWAY, True)
        vxm_ctx.sync()
    finally:
        vxm_ctx.set_path(vxm.PATH_AUTO)
    assert_trajectory_close(x.cpu().numpy(), orc.cfm_solve(ocfg, ow, x0, cond, mu, 10, 2.0, 0, 1),
                            what=f"reference cfm L=1 sway 10 steps ({path})")
    m.free()


def test_cfm_reference_shape_full_depth(vxm_ctx, orc):
    """The 12-block reference solve: its first non-zero step (sway, CFG-Zero*) within the deep-stack gross
    bar, and the full 10-step solve finite, moved and bit-identical across runs (eager then graph replays)."""
    import torch
    import vxm

    m, ow, ocfg = _model(vxm_ctx, orc, 75, **REF)
    x0, cond, mu = make_inputs(76, 4, 4, 64, 1024)
    cd, md = _dev(cond), _dev(mu)
    x = _dev(x0)
    m.cfm_solve(x, cd, md, 2, 2.0, vxm.CFM_SWAY, True)
    ref = orc.cfm_solve(ocfg, ow, x0, cond, mu, 2, 2.0, 0, 1)
    rel = np.linalg.norm(x.cpu().numpy().astype(np.float64) - ref) / np.linalg.norm(ref)
    print(f"reference cfm 12 blocks, 2 sway steps: rel_l2 {rel:.3e}")
    assert rel < 1e-1
    outs = []
    for _ in range(3):
        x = _dev(x0)
        m.cfm_solve(x, cd, md, 10, 2.0, vxm.CFM_SWAY, True)
        torch.cuda.synchronize()
        outs.append(x.cpu().numpy())
    assert np.isfinite(outs[0]).all() and not np.array_equal(outs[0], x0)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
    m.free()
