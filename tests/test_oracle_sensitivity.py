"""CPU measurements behind the full-size GPU bars (test_gpu_fullsize.py).

Two correct implementations of the path differ only in fp32 summation order.
Where that moves a value across a BF16 rounding boundary the flipped value
re-quantizes a Q8_0 block, and causal attention and the residual stream carry
the change on.  How far one such flip travels is a property of the
computation, so it is measured on the oracle itself: one input element moved
by one BF16 ulp, at the full TSLM width (hidden 2048, 16 / 2 heads of 128,
SwiGLU 6144, Q8_0 N(0, 0.02) weights from seed 1).  Each test asserts that
the GPU bar admits one flip and that the earlier, tighter bar would not.
"""
import numpy as np
import pytest

from test_gpu_fullsize import (F, H, HD, LAYER_REL, LAYER_ROW, NH, NKV, STACK_COS, STACK_REL, _prior_cache,
                               make_layers)
from test_gpu_minicpm4 import cfg_dict, layer_stats, orc_cfg, to_orc


@pytest.fixture(scope="module")
def weights():
    import vxm

    vxm.lib()
    return make_layers(vxm, 1, 28), vxm.host_randn(2, H, 1.0, 0.02)


def _bump(x, i):
    xp = x.copy()
    xp.flat[i] = np.float32(xp.flat[i] * (1 + 2.0 ** -7))   # one BF16 ulp of a BF16-range value
    return xp


def _rel_row(y, base):
    y64, b64 = np.asarray(y, np.float64), np.asarray(base, np.float64)
    rel = float(np.linalg.norm(y64 - b64) / np.linalg.norm(b64))
    row = float((np.abs(y64 - b64) / np.abs(b64).max(axis=-1, keepdims=True)).max())
    return rel, row


def test_one_flip_through_the_28_layer_decode(orc, weights):
    layers, fn = weights
    L, cap, ctx0 = 28, 512, 256
    oc = orc_cfg(orc, cfg_dict(H, L, NH, NKV, HD, F))
    ol = [to_orc(orc, d) for d in layers]
    rng = np.random.default_rng(303)
    caches = [_prior_cache(orc, rng, cap, ctx0) for _ in range(L)]
    x = rng.normal(0, 1, (1, H)).astype(np.float32)

    def run(xx, n=L, final=fn):
        return orc.minicpm4_forward(oc, ol[:n], final, xx, [k.reshape(-1).copy() for k, _ in caches[:n]],
                                    [v.reshape(-1).copy() for _, v in caches[:n]], cap, ctx0)

    base, alt = run(x), run(_bump(x, 7))
    a, b = alt.ravel().astype(np.float64), base.ravel().astype(np.float64)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
    rel = float(np.linalg.norm(a - b) / np.linalg.norm(b))
    print(f"28 layers: one flip -> rel-L2 {rel:.3g}, cos {cos:.6f}")
    assert 2e-2 < rel < STACK_REL and STACK_COS < cos < 0.9995
    # one layer: the same flip moves the block's output well past 1e-3 but within the layer bar
    rel1, row1 = _rel_row(run(_bump(x, 7), 1, None), run(x, 1, None))
    print(f"1 layer: one flip -> rel-L2 {rel1:.3g}, worst element / row max {row1:.3g}")
    assert 1e-3 < rel1 < LAYER_REL and row1 < LAYER_ROW


def test_one_flip_through_a_512_token_prefill_block(orc, weights):
    layers, _ = weights
    M, cap = 512, 512
    oc = orc_cfg(orc, cfg_dict(H, 1, NH, NKV, HD, F))
    lw = to_orc(orc, layers[0])
    x = np.random.default_rng(512).normal(0, 1, (M, H)).astype(np.float32)

    def blk(xx):
        return orc.minicpm4_block(oc, lw, xx, np.zeros(NKV * cap * HD, np.uint16),
                                  np.zeros(NKV * cap * HD, np.uint16), cap, 0, 0)

    base = blk(x)
    y = blk(_bump(x, 100 * H + 900))
    rel, row = _rel_row(y, base)
    s = layer_stats(y, base)
    changed = int((np.abs(y - base).max(axis=1) > 0).sum())
    print(f"prefill block: one flip in token 100 -> rel-L2 {rel:.3g}, worst / row max {row:.3g}, "
          f"{changed} rows changed, {s}")
    # causal attention carries it to the later tokens, past the per-element block bar
    assert changed > 300 and s["frac_ok"] < 0.99
    assert 1e-3 < rel < LAYER_REL and row < LAYER_ROW
