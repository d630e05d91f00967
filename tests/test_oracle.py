"""CPU tests that pin the oracle before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle (wrong
rounding, dropped term, transposed operand, wrong rotary pairing) fails it:
golden vectors held by the reference's own tests, library routines
(numpy / torch conversions), closed forms and brute force on tiny inputs.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

REF_FIX = os.path.join(GOLDEN, "ref_fixtures")


def _bin(name):
    return np.fromfile(os.path.join(REF_FIX, name), dtype=np.float32)


def _cos(a, b):
    a = np.ravel(a).astype(np.float64)
    b = np.ravel(b).astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


# ---------------------------------------------------------------- formats

def test_fp16_decode_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = orc.fp16_bits_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_encode_matches_numpy_rne(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # plus ties, f16 subnormal range, overflow edge, zeros
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-24, 2.0**-25, 3 * 2.0**-26,
                        2.0**-14, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 6.1e-5, -5.96e-8], dtype=np.float32)
    x = np.concatenate([x, special, rng.normal(0, 1, 100_000).astype(np.float32),
                        rng.normal(0, 1e-5, 100_000).astype(np.float32)])
    x = x[~np.isnan(x)]
    # numpy flushes nothing and rounds to nearest even; f32 denormals -> 0 in both
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    ours = orc.fp32_to_fp16_bits(x)
    assert np.array_equal(ours, ref)


def test_bf16_round_matches_torch(orc):
    import torch

    rng = np.random.default_rng(2)
    x = np.concatenate([rng.normal(0, 1, 200_000), rng.normal(0, 1e4, 50_000),
                        [1.00390625, 1.01171875, -1.00390625, 3.0e38, 0.0, -0.0]]).astype(np.float32)
    ours = orc.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------- CFM goldens

def test_cfm_sway_schedule_golden(orc):
    g = json.load(open(os.path.join(GOLDEN, "cfm_schedule.json")))
    n = g["sway_n_steps"]
    for step, want in enumerate(g["sway_expected"]):
        assert orc.sway_t(step, n) == np.float32(want), step


def test_cfm_cfg_zero_star_golden(orc):
    g = json.load(open(os.path.join(GOLDEN, "cfm_schedule.json")))
    st, v = orc.cfg_zero_star(np.array(g["cfg_negative"], np.float32), np.array(g["cfg_positive"], np.float32),
                              g["cfg_value"])
    assert st == np.float32(g["cfg_expected_scale"])
    assert np.array_equal(v, np.array(g["cfg_expected_velocity"], np.float32))


def test_cfm_zero_star_steps(orc):
    # (n+1)*0.04 truncated, at least 1 for n > 1 (src/gen_step.c:50-54)
    assert orc.zero_star_steps(1) == 0
    assert orc.zero_star_steps(10) == 1
    assert orc.zero_star_steps(49) == 2
    assert orc.zero_star_steps(100) == 4


# ---------------------------------------------------------------- Q8_0

def _blocks(q, rows, k):
    return np.asarray(q).reshape(rows, k // 32, 34)


@pytest.mark.parametrize("variant", [0, 1])
def test_quantize_invariants(orc, variant):
    rng = np.random.default_rng(3 + variant)
    rows, k = 64, 256
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    x[0, :32] = 0.0                                  # all-zero block
    q = orc.quantize_rows(x, variant)
    qs, d = orc.split_q8(q, rows, k)
    xb = x.reshape(rows, k // 32, 32)
    qb = qs.reshape(rows, k // 32, 32).astype(np.int32)
    amax = np.abs(xb).max(-1)
    dd = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(d, dd.astype(np.float16).view(np.uint16))
    assert np.all(np.abs(qb) <= 127)
    assert np.all(qb[0, 0] == 0) and d[0, 0] == 0
    # the element holding amax maps to +-127
    idx = np.abs(xb).argmax(-1)
    top = np.take_along_axis(qb, idx[..., None], -1)[..., 0]
    nz = amax > 0
    assert np.all(np.abs(top[nz]) == 127)
    # reconstruction error with the unrounded scale is at most d/2
    err = np.abs(xb - dd[..., None] * qb)
    assert np.all(err <= dd[..., None] * 0.5 * (1 + 1e-5) + 1e-12)


def test_quantize_variant_tie_known_answer(orc):
    # amax = 127 gives d = 1 and id = 1 for both variants; 2.5 and -0.5 are ties
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1] = 2.5
    x[0, 2] = -0.5
    x[0, 3] = 3.5
    ref, _ = orc.split_q8(orc.quantize_rows(x, 0), 1, 32)
    x86, _ = orc.split_q8(orc.quantize_rows(x, 1), 1, 32)
    assert list(ref[0, :4]) == [127, 3, -1, 4]      # roundf: half away from zero
    assert list(x86[0, :4]) == [127, 2, 0, 4]       # rint: half to even


def test_dequantize_round_trip(orc):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 0.02, (8, 64)).astype(np.float32)
    q = orc.quantize_rows(x, 0)
    deq = orc.dequantize_rows(q, 8, 64)
    qs, d = orc.split_q8(q, 8, 64)
    manual = qs.reshape(8, 2, 32).astype(np.float32) * d.view(np.float16).astype(np.float32)[..., None]
    assert np.array_equal(deq, manual.reshape(8, 64))
    assert np.array_equal(orc.join_q8(qs, d), q)


@pytest.mark.parametrize("N,K,M", [(1, 32, 1), (7, 64, 3), (64, 2048, 1), (5, 96, 2)])
def test_block_dots_brute_force(orc, N, K, M):
    rng = np.random.default_rng(N * 1000 + K + M)
    w = orc.quantize_rows(rng.normal(0, 0.02, (N, K)).astype(np.float32), 0)
    x = orc.quantize_rows(rng.normal(0, 1, (M, K)).astype(np.float32), 1)
    wq, _ = orc.split_q8(w, N, K)
    xq, _ = orc.split_q8(x, M, K)
    ref = np.einsum("nbj,mbj->mnb", wq.reshape(N, K // 32, 32).astype(np.int64),
                    xq.reshape(M, K // 32, 32).astype(np.int64))
    assert np.array_equal(orc.block_dots(w, x, N, K, M), ref)
    assert np.abs(ref).max() <= 32 * 127 * 128


@pytest.mark.parametrize("N,K,M", [(3, 32, 1), (16, 64, 3), (64, 2048, 2)])
def test_mul_mat_against_float64_dequant(orc, N, K, M):
    rng = np.random.default_rng(N + K * 7 + M)
    w = orc.quantize_rows(rng.normal(0, 0.02, (N, K)).astype(np.float32), 0)
    x = orc.quantize_rows(rng.normal(0, 1, (M, K)).astype(np.float32), 1)
    wq, wd = orc.split_q8(w, N, K)
    xq, xd = orc.split_q8(x, M, K)
    wf = (wq.reshape(N, K // 32, 32) * wd.view(np.float16).astype(np.float64)[..., None]).reshape(N, K)
    xf = (xq.reshape(M, K // 32, 32) * xd.view(np.float16).astype(np.float64)[..., None]).reshape(M, K)
    exact = xf @ wf.T
    y64 = orc.mul_mat_f64(w, x, N, K, M)
    y32 = orc.mul_mat(w, x, N, K, M)
    # per-block terms are fp32-rounded, so the bound scales with the row magnitude
    scale = np.abs(exact).max()
    assert np.allclose(y64, exact, rtol=1e-6, atol=1e-6 * scale)
    assert np.allclose(y32, exact, rtol=1e-4, atol=1e-5 * scale)


def test_mul_mat_identity_weight_is_dequant(orc):
    # W = I (K=N=64): y = fp32(d_w) * 127 * dequant(x) exactly per element
    K = 64
    W = np.eye(K, dtype=np.float32)
    w = orc.quantize_rows(W, 0)
    rng = np.random.default_rng(9)
    x = orc.quantize_rows(rng.normal(0, 1, (1, K)).astype(np.float32), 1)
    y = orc.mul_mat(w, x, K, K, 1)[0]
    dw = np.float32(np.float16(np.float32(1.0) / np.float32(127.0)))
    xq, xd = orc.split_q8(x, 1, K)
    want = (xq[0].astype(np.float32) * np.float32(127)) * (dw * np.repeat(xd[0].view(np.float16).astype(np.float32), 32))
    assert np.array_equal(y, want.astype(np.float32))


# ---------------------------------------------------------------- norm / rope / block

def test_rms_norm_reference_fixtures(orc):
    for name, weighted in (("rms_norm_plain", False), ("rms_norm_weighted", True)):
        x = _bin(f"{name}_input.bin").reshape(4, 8)
        gold = _bin(f"{name}_output.bin").reshape(4, 8)
        g = _bin(f"{name}_weight.bin") if weighted else None
        y = orc.rms_norm(x, g, 1e-6)
        # thresholds of tests/test_fixture_parity.c:199-204, plus BF16 elementwise bound
        assert _cos(y, gold) >= 0.9999
        assert np.sqrt(np.mean((y - gold) ** 2)) <= 0.01
        assert np.allclose(y, gold, rtol=2 ** -7, atol=0)


def test_rms_norm_known_answer(orc):
    # tests/test_minicpm4.c:154-181: [1,2,3,4] / sqrt(7.5 + 1e-6), tolerance 2e-3
    y = orc.rms_norm(np.array([[1, 2, 3, 4]], np.float32), np.ones(4, np.float32), 1e-6)[0]
    want = np.array([1, 2, 3, 4], np.float32) / np.sqrt(np.float32(7.5 + 1e-6))
    assert np.all(np.abs(y - want) <= 2e-3)


def test_rope_closed_form(orc):
    rng = np.random.default_rng(11)
    nh, hd = 3, 128
    x = orc.bf16_round(rng.normal(0, 1, nh * hd).astype(np.float32))
    # position 0 is the identity
    assert np.array_equal(orc.rope_neox(x, nh, hd, 0, 10000.0), x)
    for ff in (None, orc.ROPE_SHORT_FACTORS):
        for pos in (1, 17, 300):
            y = orc.rope_neox(x, nh, hd, pos, 10000.0, ff)
            i = np.arange(hd // 2)
            f = np.ones(hd // 2) if ff is None else ff.astype(np.float64)
            th = pos * 10000.0 ** (-2.0 * i / hd) / f
            xr = x.reshape(nh, hd).astype(np.float64)
            a, b = xr[:, : hd // 2], xr[:, hd // 2:]
            want = np.concatenate([a * np.cos(th) - b * np.sin(th), a * np.sin(th) + b * np.cos(th)], 1)
            # BF16 rounding of the output plus float32 theta accumulation
            assert np.allclose(y.reshape(nh, hd), want, rtol=1e-2, atol=2e-2), (pos, ff is None)


def test_sinusoid_closed_form(orc):
    # angle_i = 1000 t exp(-i ln(1e4) / (half - 1)); output [sin | cos].  Every
    # operand is BF16-rounded, so compare where the angle is small enough for
    # a 2^-8 relative angle error to stay below the tolerance.
    z = orc.sinusoid(0.0, 1024)
    assert np.all(z[:512] == 0) and np.all(z[512:] == 1)
    for t in (0.3, 1.0):
        e = orc.sinusoid(t, 1024)
        i = np.arange(512)
        ang = 1000.0 * t * np.exp(-i * np.log(10000.0) / 511)
        small = ang < 2.0
        assert small.sum() > 100
        # bf16(exponent) has spacing up to 2^-4 near -9, so frequencies carry up
        # to ~3.2% relative error; |d sin|, |d cos| <= |d angle|
        tol = 0.035 * ang[small] + 0.01
        assert np.all(np.abs(e[:512][small] - np.sin(ang[small])) <= tol)
        assert np.all(np.abs(e[512:][small] - np.cos(ang[small])) <= tol)


def test_mlp_reference_fixture(orc):
    x = _bin("mlp_input.bin").reshape(4, 8)
    gold = _bin("mlp_output.bin").reshape(4, 8)
    lw = orc.LayerW(wtype=1, wg=_bin("mlp_gate_weight.bin").reshape(16, 8), wu=_bin("mlp_up_weight.bin").reshape(16, 8),
                    wd=_bin("mlp_down_weight.bin").reshape(8, 16))
    cfg = orc.make_cfg(hidden=8, n_heads=1, n_kv_heads=1, head_dim=8, ffn=16)
    y = orc.mlp(cfg, lw, x)
    assert _cos(y, gold) >= 0.9999
    assert np.allclose(y, gold, rtol=2e-2)


def test_attention_reference_fixture(orc):
    # tests/fixtures/gen_op_fixtures.py:151-233: GQA 4 q heads / 2 kv heads, head_dim 4,
    # causal, no RoPE, identity-like projections stored [in][out]
    x = _bin("attention_input.bin").reshape(3, 16)
    gold = _bin("attention_output.bin").reshape(3, 16)
    wq = _bin("attention_q_weight.bin").reshape(16, 16).T
    wk = _bin("attention_k_weight.bin").reshape(16, 8).T
    wv = _bin("attention_v_weight.bin").reshape(16, 8).T
    wo = _bin("attention_o_weight.bin").reshape(16, 16).T
    lw = orc.LayerW(wtype=1, wq=wq, wk=wk, wv=wv, wo=wo)
    cfg = orc.make_cfg(hidden=16, n_heads=4, n_kv_heads=2, head_dim=4, ffn=16, no_rope=1)
    cap = 8
    kc = np.zeros(2 * cap * 4, np.uint16)
    vc = np.zeros(2 * cap * 4, np.uint16)
    y = orc.attention(cfg, lw, x, kc, vc, cap, 0, 0)
    assert _cos(y, gold) >= 0.9999
    assert np.allclose(y, gold, rtol=1e-2)
    # the GQA mapping matters: swapping kv heads must break the match
    lw2 = orc.LayerW(wtype=1, wq=wq, wk=np.roll(wk, 4, 0), wv=np.roll(wv, 4, 0), wo=wo)
    y2 = orc.attention(cfg, lw2, x, kc * 0, vc * 0, cap, 0, 0)
    assert not np.allclose(y2, gold, rtol=1e-2)


def _rand_layer(orc, rng, H, nh, nkv, hd, F):
    def q8(n, k):
        return orc.quantize_rows(rng.normal(0, 0.02, (n, k)).astype(np.float32), 0)

    return orc.LayerW(wq=q8(nh * hd, H), wk=q8(nkv * hd, H), wv=q8(nkv * hd, H), wo=q8(H, nh * hd),
                      wg=q8(F, H), wu=q8(F, H), wd=q8(H, F),
                      g_in=(1 + rng.normal(0, 0.02, H)).astype(np.float32),
                      g_post=(1 + rng.normal(0, 0.02, H)).astype(np.float32))


def test_block_prefill_equals_sequential_decode(orc):
    # Every op of the block is row-wise except attention, and causal attention
    # of token t sees exactly keys 0..t: prefill of M tokens must equal M
    # single-token decodes bit for bit.
    rng = np.random.default_rng(21)
    H, nh, nkv, hd, F, M, cap = 64, 4, 2, 16, 96, 5, 16
    lw = _rand_layer(orc, rng, H, nh, nkv, hd, F)
    cfg = orc.make_cfg(H, nh, nkv, hd, F)
    x = rng.normal(0, 1, (M, H)).astype(np.float32)
    kc = np.zeros(nkv * cap * hd, np.uint16)
    vc = np.zeros_like(kc)
    y_all = orc.minicpm4_block(cfg, lw, x, kc, vc, cap, 0, 0)
    kc2 = np.zeros_like(kc)
    vc2 = np.zeros_like(kc)
    rows = [orc.minicpm4_block(cfg, lw, x[t:t + 1], kc2, vc2, cap, t, 0) for t in range(M)]
    assert np.array_equal(y_all, np.concatenate(rows))
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


def test_block_noncausal_uses_all_tokens(orc):
    rng = np.random.default_rng(22)
    H, nh, nkv, hd, F, M = 64, 4, 4, 16, 64, 4
    lw = _rand_layer(orc, rng, H, nh, nkv, hd, F)
    cfg = orc.make_cfg(H, nh, nkv, hd, F)
    x = rng.normal(0, 1, (M, H)).astype(np.float32)
    y = orc.minicpm4_block(cfg, lw, x, None, None, 0, 0, 1)
    x2 = x.copy()
    x2[-1] += 1.0
    y2 = orc.minicpm4_block(cfg, lw, x2, None, None, 0, 0, 1)
    assert not np.allclose(y[0], y2[0])   # bidirectional: token 0 sees the last token
