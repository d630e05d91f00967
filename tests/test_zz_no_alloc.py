"""The allocation-free matmul (vxm_mul_mat_q8_0_noalloc) against the allocating
one (vxm_mul_mat_q8_0) through the C ABI.

Both run the same kernels with the same plans, so the outputs must be equal bit
for bit; each is also held to the matmul bar (1e-3 rel / 1e-4 abs of the
oracle's fp64 sum).  Every case makes two calls in a row on the shared scratch
array, the second with a smaller input, with no synchronisation in between.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _case(orc, N, K, M, seed):
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    return x, orc.quantize_rows(w, orc.QUANT_REF)


def _check(orc, vxm_ctx, wq, x, N, K, y_na, y_ref):
    assert np.array_equal(y_na, y_ref), f"noalloc differs from the allocating entry, max {np.abs(y_na - y_ref).max()}"
    xq = orc.quantize_rows(x, orc.QUANT_X86)
    ref = orc.mul_mat_f64(wq, xq, N, K, x.shape[0])
    err = np.abs(y_na.astype(np.float64) - ref)
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), f"max err {err.max()}"


# (N, K, M) pairs: the kernel the first call takes, then a smaller input
PAIRS = [
    # tiled MFMA GEMM with K split 4 ways, then the small-M GEMM with 8 K slices
    ((2048, 6144, 96), (1024, 4096, 24)),
    # small-M GEMM with K slices, then the GEMV
    ((1024, 4096, 48), (6144, 2048, 1)),
    # the same tiled product twice, fewer rows the second time (new split tags)
    ((2048, 2048, 130), (2048, 2048, 70)),
    # GEMV over two rows, then one
    ((2048, 6144, 3), (2048, 6144, 1)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_allocating_entry(vxm_ctx, orc, first, second):
    import torch

    print(f"noalloc pair {first} -> {second}", flush=True)
    runs = []
    for i, (N, K, M) in enumerate((first, second)):
        x, wq = _case(orc, N, K, M, 100 * i + N + K + M)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xd = _dev(x)
        y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda:0")
        runs.append((N, K, x, wq, w, xd, y_na))
    # the two allocation-free calls back to back on the one scratch array
    for N, K, x, wq, w, xd, y_na in runs:
        vxm_ctx.mul_mat_noalloc(w, xd, y_na)
    vxm_ctx.sync()
    outs = [r[6].cpu().numpy() for r in runs]
    for (N, K, x, wq, w, xd, _), y_na in zip(runs, outs):
        y_ref = vxm_ctx.mul_mat(w, xd).cpu().numpy()
        vxm_ctx.sync()
        _check(orc, vxm_ctx, wq, x, N, K, y_na, y_ref)
        w.free()


def test_noalloc_repeat_after_allocating_calls(vxm_ctx, orc):
    """The scratch keeps the last call's contents: a later call with new data and
    the same shape (same split tags region) still matches."""
    import torch

    N, K, M = 2048, 6144, 96
    for seed in (1, 2):
        x, wq = _case(orc, N, K, M, seed)
        w = vxm_ctx.upload_q8_0(wq, N, K)
        xd = _dev(x)
        y_ref = vxm_ctx.mul_mat(w, xd)
        y_na = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
        vxm_ctx.mul_mat_noalloc(w, xd, y_na)
        vxm_ctx.sync()
        _check(orc, vxm_ctx, wq, x, N, K, y_na.cpu().numpy(), y_ref.cpu().numpy())
        w.free()


def test_noalloc_rejects_split_above_scratch(vxm_ctx, orc):
    """2048 x 6144 at M = 520: vxm_mul_mat_q8_0 splits K 3 ways, whose partial
    words (25.6 MB) exceed the array's 16 MiB.  The allocation-free entry rejects
    the call rather than running another plan (with another summation order)."""
    import torch
    import vxm

    N, K, M = 2048, 6144, 520
    x, wq = _case(orc, N, K, M, 5)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    xd = _dev(x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
    with pytest.raises(vxm.VxmError) as e:
        vxm_ctx.mul_mat_noalloc(w, xd, y)
    assert e.value.code == 1 and "split partials" in str(e.value)
    # the allocating entry runs the split plan; it stays within the matmul bar
    y_ref = vxm_ctx.mul_mat(w, xd).cpu().numpy()
    vxm_ctx.sync()
    xq = orc.quantize_rows(x, orc.QUANT_X86)
    ref = orc.mul_mat_f64(wq, xq, N, K, M)
    err = np.abs(y_ref.astype(np.float64) - ref)
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), f"max err {err.max()}"
    w.free()


def test_noalloc_rejects_oversize(vxm_ctx, orc):
    import torch
    import vxm

    assert vxm.lib().vxm_noalloc_scratch_bytes() == (48 << 20) + (64 << 10)
    N, K, M = 64, 8192, 4096   # quantized activation 35.7 MB > 32 MiB
    _, wq = _case(orc, N, K, 1, 3)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    x = torch.zeros((M, K), dtype=torch.float32, device="cuda:0")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
    with pytest.raises(vxm.VxmError) as e:
        vxm_ctx.mul_mat_noalloc(w, x, y)
    assert e.value.code == 1 and "scratch" in str(e.value)
    w.free()
