"""GPU parity of the Q8_0 matmul path against the CPU oracle.

Bar: quantized activations and int32 per-block sums bit-exact; fp32 outputs
within 1e-3 relative / 1e-4 absolute of the oracle's fp64 sum of the same
per-block terms (the GPU adds the terms in a different order than ggml).
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _np(t):
    return t.cpu().numpy()


def _case(orc, N, K, M, seed, wstd=0.02):
    rng = np.random.default_rng(seed)
    w = rng.normal(0, wstd, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    return w, x, orc.quantize_rows(w, orc.QUANT_REF)


def _assert_close(y, ref64):
    err = np.abs(y.astype(np.float64) - ref64)
    bad = err > ATOL + RTOL * np.abs(ref64)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside 1e-3 rel / 1e-4 abs, max err {err.max()}"


def test_upload_download_round_trip(vxm_ctx, orc):
    for N, K in ((1, 32), (7, 96), (33, 2048), (5, 6144)):
        _, _, wq = _case(orc, N, K, 1, N + K)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        assert np.array_equal(w.download(), wq)
        w.free()


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("M,K", [(1, 32), (3, 64), (1, 2048), (2, 6144), (17, 1024)])
def test_quantize_bit_exact(vxm_ctx, orc, variant, M, K):
    rng = np.random.default_rng(M * 31 + K + variant)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    x[0, :32] = 0.0                       # zero block
    if K >= 64:
        x[0, 32:64] = np.arange(32) - 15.5   # exact halves after scaling
        x[0, 63] = 127.0
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), variant)
    ref = orc.quantize_rows(x, variant)
    qs, d = orc.split_q8(ref, M, K)
    assert np.array_equal(_np(xq), qs)
    assert np.array_equal(_np(xd).view(np.uint16), d)


@pytest.mark.parametrize("N,K,M", [(1, 32, 1), (7, 64, 3), (5, 96, 2), (64, 1024, 1), (33, 2048, 2),
                                   (16, 6144, 1), (9, 4096, 3), (4, 3072, 1)])
def test_block_dots_bit_exact(vxm_ctx, orc, N, K, M):
    _, x, wq = _case(orc, N, K, M, 7 * N + K + M)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    got = _np(vxm_ctx.block_dots(w, xq, xd))
    ref = orc.block_dots(wq, orc.quantize_rows(x, 1), N, K, M)
    assert np.array_equal(got, ref)
    w.free()


@pytest.mark.parametrize("N,K,M", [(1, 32, 1), (7, 64, 3), (5, 96, 2), (257, 512, 1), (64, 1024, 1),
                                   (130, 2048, 1), (33, 2048, 3), (16, 6144, 2), (9, 4096, 1),
                                   (4, 3072, 2), (1000, 1024, 4)])
def test_mul_mat_matches_oracle(vxm_ctx, orc, N, K, M):
    _, x, wq = _case(orc, N, K, M, 11 * N + K + M)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    y = _np(vxm_ctx.mul_mat(w, _dev(x)))
    xq = orc.quantize_rows(x, 1)
    _assert_close(y, orc.mul_mat_f64(wq, xq, N, K, M))
    # and against ggml's sequential fp32 order
    _assert_close(y, orc.mul_mat(wq, xq, N, K, M).astype(np.float64))
    w.free()


def test_golden_cases(vxm_ctx, orc):
    g = np.load(os.path.join(GOLDEN, "q8_cases.npz"))
    i = 0
    while f"c{i}_shape" in g:
        N, K, M = (int(v) for v in g[f"c{i}_shape"])
        w = vxm_ctx.upload_q8_0(g[f"c{i}_wq"], N, K)
        xq, xd = vxm_ctx.quantize_q8_0(_dev(g[f"c{i}_x"]), 1)
        qs, d = orc.split_q8(g[f"c{i}_xq"], M, K)
        assert np.array_equal(_np(xq), qs) and np.array_equal(_np(xd).view(np.uint16), d)
        assert np.array_equal(_np(vxm_ctx.block_dots(w, xq, xd)), g[f"c{i}_sums"])
        _assert_close(_np(vxm_ctx.mul_mat_q8(w, xq, xd)), g[f"c{i}_y64"])
        w.free()
        i += 1
    assert i == 6


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144)])
def test_decode_gemv_full_size_seed0(vxm_ctx, orc, N, K):
    """The GEMV workload: W ~ N(0, 0.02) from seed 0, x ~ N(0, 1), Q8_0 both."""
    import vxm

    w32 = vxm.host_randn(0, N * K, 0.0, 0.02).reshape(N, K)
    x = vxm.host_randn(0, K, 0.0, 1.0, offset=N * K).reshape(1, K)
    wq = vxm.host_quantize_q8_0(w32)
    assert np.array_equal(wq[: 34 * (K // 32)], orc.quantize_rows(w32[:1], orc.QUANT_REF))
    w = vxm_ctx.upload_q8_0(wq, N, K)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    xq_ref = orc.quantize_rows(x, 1)
    # every int32 block sum bit-exact
    assert np.array_equal(_np(vxm_ctx.block_dots(w, xq, xd)), orc.block_dots(wq, xq_ref, N, K, 1))
    y = _np(vxm_ctx.mul_mat_q8(w, xq, xd))
    _assert_close(y, orc.mul_mat_f64(wq, xq_ref, N, K, 1))
    w.free()


# (path, N, K, M): the kernel vxm_mul_mat_q8_0_q8_0 runs for each is the one whose
# int32 block sums vxm_block_dots_q8_0 returns -- chunked GEMV <C, R> (M < 8, K a
# multiple of 1024 in {1, 2, 4, 6} KiB), generic GEMV, small-M MFMA (one or two wave
# groups, K splits), the DMA-fed tile GEMM (64 x 64, 64 x 128 or 128 x 128 tiles,
# K % 256 == 0, K splits), the register-staged tiled GEMM (16- or 8-block stages, K splits)
_PRODUCTION_DOTS = [
    (0, 6144, 2048, 1),     # decode gate/up GEMV <2, 2>
    (0, 2048, 6144, 1),     # decode down GEMV <6, 1>
    (0, 2560, 2048, 3),     # GEMV <2, 2>, three activation rows
    (0, 1024, 4096, 5),     # LocEnc down at 5 rows: GEMV <4, 1>
    (0, 256, 1024, 2),      # GEMV <1, 4>
    (0, 7, 96, 2),          # generic GEMV
    (0, 8192, 1024, 48),    # CFM gate/up at 2 x 24 rows: small-M
    (0, 3072, 1024, 48),    # CFM QKV: small-M
    (0, 1024, 4096, 48),    # CFM down: small-M, K split
    (2, 1024, 4096, 5),     # small-M at 5 rows (the block pipeline's choice)
    (0, 2048, 2048, 512),   # prefill O: tile GEMM, 64 x 64 tiles
    (0, 2560, 1024, 512),   # tile GEMM, 64 x 128 tiles (the prefill QKV choice)
    (0, 8192, 256, 512),    # tile GEMM, 128 x 128 tiles (one full round of 256; long-prompt gate/up, O)
    (0, 256, 8192, 128),    # tile GEMM, four K splits (more blocks than one activation scale panel holds)
    (0, 1001, 512, 100),    # tile GEMM, ragged M and N (N % 4 != 0: no 16-byte stores)
    (3, 2048, 2048, 33),    # tiled, 16-block stages, K split
    (0, 2560, 2048, 100),   # tile GEMM, ragged M tile
    (0, 2560, 2080, 100),   # register-staged tiled GEMM (K % 256 != 0)
]


@pytest.mark.parametrize("path,N,K,M", _PRODUCTION_DOTS)
def test_block_dots_of_the_kernel_that_runs(vxm_ctx, orc, path, N, K, M):
    """The int32 block sums of the kernel the matmul dispatch picks are bit-exact,
    and that kernel's fp32 output is the oracle combine of exactly these sums."""
    _, x, wq = _case(orc, N, K, M, 5 * N + K + 3 * M)
    vxm_ctx.set_path(path)
    try:
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
        sums = _np(vxm_ctx.block_dots(w, xq, xd))
        y = _np(vxm_ctx.mul_mat_q8(w, xq, xd))
        vxm_ctx.sync()
    finally:
        vxm_ctx.set_path(0)
    xq_ref = orc.quantize_rows(x, 1)
    assert np.array_equal(sums, orc.block_dots(wq, xq_ref, N, K, M))
    # y = sum_b sumi * (d_w * d_x) over the device's own sums, in fp64
    _, dw = orc.split_q8(wq, N, K)
    _, dx = orc.split_q8(xq_ref, M, K)
    scale = (dx.view(np.float16).astype(np.float32)[:, None, :] * dw.view(np.float16).astype(np.float32)[None, :, :])
    terms = (sums.astype(np.float32) * scale).astype(np.float64)
    _assert_close(y, terms.sum(axis=2))
    w.free()


@pytest.mark.parametrize("N,K,M", [(2048, 2048, 512), (2560, 1024, 512), (8192, 256, 512), (256, 8192, 128),
                                   (1001, 512, 100), (8192, 1024, 48)])
def test_gemm_subnormal_scales(vxm_ctx, orc, N, K, M):
    """Every third weight row and every other activation row are scaled so far down that
    each of their Q8_0 scales is an fp16 subnormal (block maxima near 3e-5, d near 2e-7).
    The scale products d_x * d_w must still be the exact fp32 products: each output is
    the fp64 combine of the kernel's own int32 block sums to within fp32 summation error
    (a subnormal scale flushed to zero would zero whole rows)."""
    rng = np.random.default_rng(3 * N + K + M)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    w[::3] *= 5e-4
    x[::2] *= 1e-5
    wq = orc.quantize_rows(w, orc.QUANT_REF)
    _, dw = orc.split_q8(wq, N, K)
    dwf = dw.view(np.float16).astype(np.float32)
    assert (np.abs(dwf[::3]) < 2.0 ** -14).all() and (dwf[::3] != 0).any()
    w_dev = vxm_ctx.upload_q8_0(wq, N, K)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    sums = _np(vxm_ctx.block_dots(w_dev, xq, xd))
    y = _np(vxm_ctx.mul_mat_q8(w_dev, xq, xd))
    vxm_ctx.sync()
    xq_ref = orc.quantize_rows(x, 1)
    assert np.array_equal(sums, orc.block_dots(wq, xq_ref, N, K, M))
    _, dx = orc.split_q8(xq_ref, M, K)
    dxf = dx.view(np.float16).astype(np.float32)
    assert (np.abs(dxf[::2]) < 2.0 ** -14).all()
    terms = (sums.astype(np.float32) * (dxf[:, None, :] * dwf[None, :, :])).astype(np.float64)
    ref, mag = terms.sum(axis=2), np.abs(terms).sum(axis=2)
    err = np.abs(y.astype(np.float64) - ref)
    assert (err <= 1e-5 * mag + 1e-30).all(), f"max err / magnitude {(err / np.maximum(mag, 1e-300)).max()}"
    assert (y[::2][:, ::3] != 0).mean() > 0.9   # the subnormal x subnormal products are not flushed
    w_dev.free()


def test_tile_gemm_unaligned_output(vxm_ctx, orc):
    """An output pointer that is 4- but not 16-byte aligned takes the tile GEMM's
    scalar stores: the same bits as into an aligned buffer."""
    import torch

    N, K, M = 640, 1024, 256
    _, x, wq = _case(orc, N, K, M, 91)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    y_al = vxm_ctx.mul_mat_q8(w, xq, xd)
    buf = torch.full((M * N + 1,), float("nan"), dtype=torch.float32, device=xq.device)
    y_un = buf[1:].view(M, N)
    assert y_un.data_ptr() % 16 != 0
    vxm_ctx.mul_mat_q8(w, xq, xd, y_un)
    vxm_ctx.sync()
    assert torch.equal(y_al, y_un)
    assert torch.isnan(buf[0])   # nothing written before the output
    w.free()


@pytest.fixture
def mfma_path(vxm_ctx):
    import vxm

    vxm_ctx.set_path(vxm.PATH_MFMA)
    yield vxm_ctx
    vxm_ctx.set_path(vxm.PATH_AUTO)


# Shapes whose MFMA GEMM runs without a K split on a 256-CU device: either fewer than
# 8 blocks per row (no split is ever taken) or at least 256 64x64 output tiles.
@pytest.mark.parametrize("N,K,M", [(100, 224, 70), (300, 128, 200), (64, 32, 1), (1024, 192, 512),
                                   (2048, 6144, 512), (6144, 2048, 256), (4096, 256, 300)])
def test_mfma_gemm_unsplit(mfma_path, orc, N, K, M):
    """The MFMA's own int32 block sums are bit-exact (ggml's vec_dot_q8_0_q8_0 per block);
    the scaled fp32 outputs meet the oracle bar against the fp64 and the sequential sums."""
    ctx = mfma_path
    _, x, wq = _case(orc, N, K, M, 13 * N + K + M)
    w = ctx.upload_q8_0(wq, N, K)
    xq_d, xd_d = ctx.quantize_q8_0(_dev(x), 1)
    xq = orc.quantize_rows(x, 1)
    if M * N * (K // 32) <= 1 << 23:
        assert np.array_equal(_np(ctx.block_dots(w, xq_d, xd_d)), orc.block_dots(wq, xq, N, K, M))
    y = _np(ctx.mul_mat_q8(w, xq_d, xd_d))
    _assert_close(y, orc.mul_mat_f64(wq, xq, N, K, M))
    _assert_close(y, orc.mul_mat(wq, xq, N, K, M).astype(np.float64))
    w.free()


# Small-M shapes (CFM / short prefill) where the K dimension is split to fill the device.
@pytest.mark.parametrize("N,K,M", [(1024, 1024, 48), (2560, 2048, 16), (6144, 2048, 8), (2048, 6144, 48),
                                   (1000, 4096, 100), (33, 2048, 3), (130, 1024, 9)])
def test_mfma_gemm_split_k(mfma_path, orc, N, K, M):
    ctx = mfma_path
    _, x, wq = _case(orc, N, K, M, 17 * N + K + M)
    w = ctx.upload_q8_0(wq, N, K)
    xq_d, xd_d = ctx.quantize_q8_0(_dev(x), 1)
    y = _np(ctx.mul_mat_q8(w, xq_d, xd_d))
    xq = orc.quantize_rows(x, 1)
    _assert_close(y, orc.mul_mat_f64(wq, xq, N, K, M))
    _assert_close(y, orc.mul_mat(wq, xq, N, K, M).astype(np.float64))
    # the exact block sums do not depend on the path
    assert np.array_equal(_np(ctx.block_dots(w, xq_d, xd_d)), orc.block_dots(wq, xq, N, K, M))
    w.free()


# Shapes of the register-fed small-M MFMA kernel (M <= 64, N % 64 == 0, K % 512 == 0):
# the LocDiT projections at M = 2 x 24, a single 64-row group, partial m-tiles, one
# 16-block stage, several stages per split (long K) and 2 to 8 K splits.  The tiled GEMM (forced) must meet the same bar on the same inputs.
@pytest.mark.parametrize("N,K,M", [(8192, 1024, 48), (3072, 1024, 48), (1024, 1024, 48), (1024, 4096, 48),
                                   (2048, 6144, 48), (64, 512, 5), (64, 32768, 64), (2560, 2048, 16),
                                   (6144, 2048, 8), (128, 1536, 33), (1024, 512, 1), (4096, 1024, 64)])
def test_mfma_small_m(vxm_ctx, orc, N, K, M):
    import vxm

    _, x, wq = _case(orc, N, K, M, 19 * N + K + M)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    xq_d, xd_d = vxm_ctx.quantize_q8_0(_dev(x), 1)
    ref = orc.mul_mat_f64(wq, orc.quantize_rows(x, 1), N, K, M)
    try:
        vxm_ctx.set_path(vxm.PATH_MFMA)
        y = _np(vxm_ctx.mul_mat_q8(w, xq_d, xd_d))
        _assert_close(y, ref)
        # the split reduction adds in a fixed order: a repeat is bit-identical
        assert np.array_equal(y, _np(vxm_ctx.mul_mat_q8(w, xq_d, xd_d)))
        vxm_ctx.set_path(vxm.PATH_MFMA_TILED)
        _assert_close(_np(vxm_ctx.mul_mat_q8(w, xq_d, xd_d)), ref)
    finally:
        vxm_ctx.set_path(vxm.PATH_AUTO)
    w.free()


def test_mfma_small_m_back_to_back_shapes(vxm_ctx, orc):
    """Consecutive split launches of different shapes share the tagged partial buffer:
    each must read only its own launch's words."""
    cases = []
    for (N, K, M) in ((1024, 4096, 48), (1024, 1024, 40), (1024, 4096, 48), (3072, 1024, 24)):
        _, x, wq = _case(orc, N, K, M, 7 * N + 3 * K + M)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xq_d, xd_d = vxm_ctx.quantize_q8_0(_dev(x), 1)
        cases.append((w, xq_d, xd_d, orc.mul_mat_f64(wq, orc.quantize_rows(x, 1), N, K, M)))
    ys = [vxm_ctx.mul_mat_q8(w, a, b) for (w, a, b, _) in cases]
    for y, (w, _, _, ref) in zip(ys, cases):
        _assert_close(_np(y), ref)
        w.free()


def test_auto_path_switches_at_eight_rows(vxm_ctx, orc):
    """AUTO takes the GEMV below 8 rows and the MFMA GEMM from 8; both meet the oracle bar
    and the repeated call is deterministic."""
    import vxm

    N, K = 2048, 2048
    for M in (7, 8, 64):
        _, x, wq = _case(orc, N, K, M, M)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xd = _dev(x)
        y_auto = _np(vxm_ctx.mul_mat(w, xd))
        assert np.array_equal(y_auto, _np(vxm_ctx.mul_mat(w, xd)))
        vxm_ctx.set_path(vxm.PATH_GEMV)
        y_gemv = _np(vxm_ctx.mul_mat(w, xd))
        vxm_ctx.set_path(vxm.PATH_MFMA)
        y_mfma = _np(vxm_ctx.mul_mat(w, xd))
        vxm_ctx.set_path(vxm.PATH_AUTO)
        assert np.array_equal(y_auto, y_gemv if M < 8 else y_mfma)
        ref = orc.mul_mat_f64(wq, orc.quantize_rows(x, 1), N, K, M)
        _assert_close(y_gemv, ref)
        _assert_close(y_mfma, ref)
        w.free()


# (K, [N of each product], M): products of one K in one launch
_MULTI = [
    (2048, [2048, 256, 256, 6144, 12288], 1),   # q, k, v, gate, gate/up-sized
    (6144, [2048, 2048, 64], 1),                # down-sized
    (1024, [1024, 37, 3072], 2),                # GEMV <1, 4> with a ragged N
    (4096, [1024, 5], 3),                       # GEMV <4, 1>, three rows
    (96, [7, 5], 2),                            # K outside the chunked GEMV: one launch each
]


@pytest.mark.parametrize("K,Ns,M", _MULTI)
def test_mul_mat_multi_bit_identical_to_single(vxm_ctx, orc, K, Ns, M):
    """Every output of the one-launch GEMV batch equals the single GEMV's bit for
    bit (the same per-wave code), and the single GEMV's block sums are pinned."""
    import torch

    ws, xqs, xds, singles, refs = [], [], [], [], []
    for i, N in enumerate(Ns):
        _, x, wq = _case(orc, N, K, M, 1000 + 17 * i + K + M)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
        ws.append(w); xqs.append(xq); xds.append(xd)
        singles.append(_np(vxm_ctx.mul_mat_q8(w, xq, xd)))
        refs.append(orc.mul_mat_f64(wq, orc.quantize_rows(x, 1), N, K, M))
    ys = [torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda:0") for N in Ns]
    vxm_ctx.mul_mat_q8_multi(ws, xqs, xds, ys)
    for y, s, r in zip(ys, singles, refs):
        got = _np(y)
        assert np.array_equal(got.view(np.uint32), s.view(np.uint32))
        _assert_close(got, r)
    for w in ws:
        w.free()


def test_mul_mat_multi_more_than_one_launch(vxm_ctx, orc):
    """70 products (a launch takes 64): every output still equals the single GEMV's."""
    import torch

    N, K, M = 128, 2048, 1
    _, x, _ = _case(orc, 1, K, M, 5)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    ws, ys, singles = [], [], []
    for i in range(70):
        _, _, wq = _case(orc, N, K, 1, 300 + i)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        ws.append(w)
        singles.append(_np(vxm_ctx.mul_mat_q8(w, xq, xd)))
        ys.append(torch.empty((M, N), dtype=torch.float32, device="cuda:0"))
    vxm_ctx.mul_mat_q8_multi(ws, [xq] * 70, [xd] * 70, ys)
    for y, s in zip(ys, singles):
        assert np.array_equal(_np(y).view(np.uint32), s.view(np.uint32))
    for w in ws:
        w.free()


def test_mul_mat_multi_rejects_mixed_k(vxm_ctx, orc):
    import vxm

    _, x, wq1 = _case(orc, 64, 1024, 1, 1)
    _, _, wq2 = _case(orc, 64, 2048, 1, 2)
    w1, w2 = vxm_ctx.upload_q8_0(wq1, 64, 1024), vxm_ctx.upload_q8_0(wq2, 64, 2048)
    xq, xd = vxm_ctx.quantize_q8_0(_dev(x), 1)
    import torch

    ys = [torch.empty((1, 64), dtype=torch.float32, device="cuda:0") for _ in range(2)]
    with pytest.raises(vxm.VxmError) as e:
        vxm_ctx.mul_mat_q8_multi([w1, w2], [xq, xq], [xd, xd], ys)
    assert e.value.code == 1
    w1.free()
    w2.free()


def test_stream_read_checksum(vxm_ctx):
    """The read floor kernel reads every byte once: its XOR of all 32-bit words
    equals numpy's over the same ranges (ragged sizes, several ranges)."""
    import torch

    rng = np.random.default_rng(9)
    sizes = [16, 16384, 16400, 1 << 20, 13369344 + 16 * 7]
    hs = [rng.integers(0, 2 ** 32, n // 4, dtype=np.uint32) for n in sizes]
    ds = [torch.from_numpy(h.view(np.int32)).to("cuda:0") for h in hs]
    sink = vxm_ctx.stream_read(ds)
    vxm_ctx.sync()
    ref = np.uint32(0)
    for h in hs:
        ref ^= np.bitwise_xor.reduce(h)
    assert int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))) == int(ref)


@pytest.mark.parametrize("nbytes,offset", [(8192, 0), (16, 0), (65536, 0), (65552, 0), (8192, 4), (100, 0), (96, 16)])
def test_memcpy_d2h_sizes(vxm_ctx, nbytes, offset):
    """vxm_memcpy_d2h returns exactly the device bytes: small 16-byte-aligned copies
    through the pinned staging buffer (the per-token hidden state), larger, unaligned
    or ragged ones through the DMA copy; twice in a row with new contents."""
    import ctypes
    import torch
    import vxm

    for rep in range(2):
        src = torch.randint(0, 256, (nbytes + offset,), dtype=torch.uint8, device="cuda:0")
        want = src.cpu().numpy()[offset:]
        got = np.full(nbytes, 0xA5, dtype=np.uint8)
        vxm_ctx.check(
            vxm.lib().vxm_memcpy_d2h(vxm_ctx.h, got.ctypes.data_as(ctypes.c_void_p),
                                         ctypes.c_void_p(src.data_ptr() + offset), nbytes))
        assert np.array_equal(got, want), (nbytes, offset, rep)
