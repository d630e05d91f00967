"""HIP graph capture of K-split matmuls through the C ABI (vxm_capture_begin /
vxm_capture_end / vxm_graph_launch).

The tiled GEMM's K splits hand partial tiles to the tile's last workgroup as
tagged words.  The tag is a device word advanced before every split launch, so a
graph replay reads a tag no earlier launch used.  With a host-side tag, a
captured launch would replay one fixed tag, and the last workgroup of a tile
could take a partial word that the previous replay left behind.

Each test records vxm_mul_mat_q8_0 and vxm_mul_mat_q8_0_noalloc on a shape whose
plan splits K (2048 x 6144 from 96 rows: 4 splits), then replays the graph three
times with new activations written into the same device buffer, with eager work
between the replays.  Every replay must equal an eager call on the same inputs
bit for bit, and the oracle's fp64 product to the matmul bar.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def _wq(orc, N, K, seed):
    rng = np.random.default_rng(seed)
    return orc.quantize_rows(rng.normal(0, 0.02, (N, K)).astype(np.float32), orc.QUANT_REF)


def _bar(orc, wq, x, N, K, y):
    xq = orc.quantize_rows(x, orc.QUANT_X86)
    ref = orc.mul_mat_f64(wq, xq, N, K, x.shape[0])
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= ATOL + RTOL * np.abs(ref)), f"max err {err.max()}"


@pytest.mark.parametrize("N,K,M", [(2048, 6144, 96), (2048, 2048, 130)])
def test_captured_split_matmul_replays_match_eager(vxm_ctx, orc, N, K, M):
    import torch

    print(f"graph capture of split matmuls {N}x{K} M={M}", flush=True)
    wq = _wq(orc, N, K, 7)
    w = vxm_ctx.upload_q8_0(wq, N, K)
    x_dev = torch.zeros((M, K), dtype=torch.float32, device="cuda:0")
    y_cap = torch.zeros((M, N), dtype=torch.float32, device="cuda:0")
    y_cap_na = torch.zeros((M, N), dtype=torch.float32, device="cuda:0")
    # eager once first: every scratch buffer the sequence needs exists before capture
    vxm_ctx.mul_mat(w, x_dev, y_cap)
    vxm_ctx.mul_mat_noalloc(w, x_dev, y_cap_na)
    vxm_ctx.sync()
    vxm_ctx.capture_begin()
    try:
        vxm_ctx.mul_mat(w, x_dev, y_cap)
        vxm_ctx.mul_mat_noalloc(w, x_dev, y_cap_na)
    finally:
        g = vxm_ctx.capture_end()
    try:
        rng = np.random.default_rng(11)
        for rep in range(3):
            x = rng.normal(0, 1, (M, K)).astype(np.float32)
            x_dev.copy_(torch.from_numpy(x))
            torch.cuda.synchronize()
            # eager work on the same scratch between the replays (advances the tag word)
            y_eager = vxm_ctx.mul_mat(w, x_dev)
            y_eager_na = torch.empty_like(y_eager)
            vxm_ctx.mul_mat_noalloc(w, x_dev, y_eager_na)
            y_cap.fill_(float("nan"))
            y_cap_na.fill_(float("nan"))
            torch.cuda.synchronize()
            g.launch()
            vxm_ctx.sync()
            ye, yen = y_eager.cpu().numpy(), y_eager_na.cpu().numpy()
            yc, ycn = y_cap.cpu().numpy(), y_cap_na.cpu().numpy()
            assert np.array_equal(ye, yen), f"replay {rep}: eager noalloc differs from eager allocating"
            assert np.array_equal(yc, ye), f"replay {rep}: captured allocating entry differs from eager"
            assert np.array_equal(ycn, ye), f"replay {rep}: captured noalloc entry differs from eager"
            _bar(orc, wq, x, N, K, yc)
    finally:
        g.free()
        w.free()


def test_capture_refuses_scratch_growth(vxm_ctx, orc):
    """A call that would have to grow a scratch buffer under capture fails with
    a clear error instead of allocating into the recorded stream (a fresh
    context: its activation scratch starts empty)."""
    import torch
    import vxm

    N, K, M = 1024, 4096, 96
    with vxm.Context(0) as ctx:
        w = ctx.upload_q8_0(_wq(orc, N, K, 8), N, K)
        x = torch.zeros((M, K), dtype=torch.float32, device="cuda:0")
        y = torch.empty((M, N), dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        ctx.capture_begin()
        err = None
        try:
            ctx.mul_mat(w, x, y)
        except vxm.VxmError as e:
            err = e
        finally:
            try:
                ctx.capture_end().free()
            except vxm.VxmError:
                pass   # the capture recorded nothing
        assert err is not None and err.code == 1 and "capture" in str(err), err
        # the context still works afterwards, and then captures the same call
        ctx.mul_mat(w, x, y)
        ctx.sync()
        ctx.capture_begin()
        try:
            ctx.mul_mat(w, x, y)
        finally:
            g = ctx.capture_end()
        g.launch()
        ctx.sync()
        g.free()
        w.free()


def test_capture_refuses_first_single_launch_blocks(orc):
    """The single-launch LocEnc blocks set up their exchange buffers and block table
    on their first eager evaluation; captured before that, the call fails with a
    clear error (nothing is allocated into the recording), and after one eager
    evaluation the same call captures and replays bit-identically, tagging anew
    on every replay."""
    import torch
    import vxm
    from test_lm_update_host import make_locenc

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")

    with vxm.Context(0) as ctx:
        cfg, w, _, _ = make_locenc(orc, 813, H=1024, L=2, nh=16, nkv=2, hd=128, F=4096, special=True)
        enc = vxm.LocEnc(ctx, cfg, w)
        x = dev(np.random.default_rng(814).normal(0, 1, (4, 64)).astype(np.float32))
        out = torch.full((1024,), float("nan"), dtype=torch.float32, device="cuda:0")
        try:
            # one evaluation launch by launch: the context's scratch and the encoder's own
            # buffers exist, the single launch's buffers do not yet
            enc.set_block_mode(vxm.DECODE_KERNELS)
            enc.forward(x, out)
            ctx.sync()
            enc.set_block_mode(vxm.DECODE_PERSISTENT)
            ctx.capture_begin()
            err = None
            try:
                enc.forward(x, out)
            except vxm.VxmError as e:
                err = e
            finally:
                try:
                    ctx.capture_end().free()
                except vxm.VxmError:
                    pass
            assert err is not None and err.code == 1 and "persistent blocks" in str(err) and "eager" in str(err), err
            ref = enc.forward(x).cpu().numpy()   # eager: sets up the single launch's buffers
            enc.check()
            ctx.capture_begin()
            try:
                enc.forward(x, out)
            finally:
                g = ctx.capture_end()
            try:
                for _ in range(3):
                    out.fill_(float("nan"))
                    torch.cuda.synchronize()
                    g.launch()
                    ctx.sync()
                    assert np.array_equal(out.cpu().numpy(), ref)
                    enc.check()
                    # eager launches between replays advance the same device epoch
                    assert np.array_equal(enc.forward(x).cpu().numpy(), ref)
            finally:
                g.free()
        finally:
            enc.free()
