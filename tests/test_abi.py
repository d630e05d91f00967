"""CPU tests of the C ABI library: it loads, exports every declared symbol,
and its host-only helpers agree with the oracle.  No device work here."""
import os

import numpy as np

from conftest import GOLDEN, ROOT


def test_library_exports_every_header_symbol():
    import vxm

    names = vxm.header_functions()
    assert len(names) >= 20
    L = vxm.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the Python mirror binds every declared function with a signature
    assert set(names) <= set(vxm._SIGS), set(names) - set(vxm._SIGS)


def test_open_without_device_fails_cleanly():
    import torch
    import vxm

    if torch.cuda.is_available():
        return  # on a GPU host opening succeeds; covered by the gpu tests
    try:
        vxm.Context(0)
    except vxm.VxmError as e:
        assert e.code in (4, 5)
    else:
        raise AssertionError("vxm_open succeeded without a device")


def test_host_quantize_matches_oracle(orc):
    import vxm

    rng = np.random.default_rng(7)
    x = rng.normal(0, 0.02, (33, 256)).astype(np.float32)
    x[3, 32:64] = 0.0
    assert np.array_equal(vxm.host_quantize_q8_0(x), orc.quantize_rows(x, orc.QUANT_REF))


def test_host_quantize_golden():
    import vxm

    g = np.load(os.path.join(GOLDEN, "q8_cases.npz"))
    for i in range(6):
        if f"c{i}_w" in g:
            assert np.array_equal(vxm.host_quantize_q8_0(g[f"c{i}_w"]), g[f"c{i}_wq"])


def test_host_randn_is_seeded_sliceable_and_normal():
    import vxm

    a = vxm.host_randn(0, 100_001, 0.0, 1.0)
    b = vxm.host_randn(0, 100_001, 0.0, 1.0)
    assert np.array_equal(a, b)
    # any slice is reproducible on its own
    assert np.array_equal(vxm.host_randn(0, 1000, 0.0, 1.0, offset=4321), a[4321:5321])
    assert np.array_equal(vxm.host_randn(0, 7, 0.0, 1.0, offset=99_990), a[99_990:99_997])
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1.0) < 0.02
    c = vxm.host_randn(1, 100_000, 0.0, 0.02)
    assert abs(c.std() - 0.02) < 0.001
    assert not np.array_equal(c[:10] / 0.02, a[:10])
    # first values are the Box-Muller pair of SplitMix64 outputs 1 and 2
    G = 0x9E3779B97F4A7C15
    M64 = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    u1 = ((mix(G) >> 11) + 1) * 2.0 ** -53
    u2 = (mix(2 * G & M64) >> 11) * 2.0 ** -53
    r = np.sqrt(-2 * np.log(u1))
    assert a[0] == np.float32(r * np.cos(2 * np.pi * u2))
    assert a[1] == np.float32(r * np.sin(2 * np.pi * u2))


def test_graft_entry_has_build_and_smoke():
    import importlib.util

    spec = importlib.util.spec_from_file_location("ge", os.path.join(ROOT, "__graft_entry__.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    assert callable(m.build) and callable(m.smoke)
