"""Packs the reference's weight-free CFM / LocDiT-time fixtures into ref_cfm.npz.

Source: the reference's PyTorch intermediates fixtures/ref/ar%04d_d%04d_*.npy (float32 .npy,
read with numpy.load(allow_pickle=False)) for utterances 0 and 1 of its AR run: the CFM
trajectory states, the cond / uncond / blended velocities and CFG-Zero* st* of every Euler
step, and the LocDiT time pieces of each step (sinusoids of t and dt, the two time-MLP
outputs and their BF16 sum).  Only data is copied.  Run here, where the reference tree is
mounted:  python tests/golden/pack_ref_cfm.py /root/reference
"""
import os
import sys

import numpy as np

PIECES = ("cfm_traj_state", "cfm_velocity_cond", "cfm_velocity_uncond", "cfm_velocity_blend", "cfm_cfg_st_star",
          "locdit_cond_t_sin", "locdit_cond_dt_sin", "locdit_cond_t_feat", "locdit_cond_dt_feat",
          "locdit_cond_t_combined", "locdit_uncond_t_sin", "locdit_uncond_t_combined")


def main(ref_root):
    src = os.path.join(ref_root, "fixtures", "ref")
    out = {}
    for ar in (0, 1):
        for name in ("cfm_noise", "cfm_clean"):
            out[f"ar{ar}_{name}"] = np.load(os.path.join(src, f"ar{ar:04d}_{name}.npy"), allow_pickle=False)
        for d in range(0, 11):
            for piece in PIECES:
                f = os.path.join(src, f"ar{ar:04d}_d{d:04d}_{piece}.npy")
                if os.path.exists(f):
                    out[f"ar{ar}_d{d}_{piece}"] = np.load(f, allow_pickle=False).astype(np.float32)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_cfm.npz")
    np.savez_compressed(dst, **out)
    print(f"{len(out)} arrays -> {dst} ({os.path.getsize(dst)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
