"""Per-phase timeline of the single-launch decode from the profiling build's traces.

The profiling build (`make -C voxcpm-cpp_amd trace`, loaded with VXM_LIB=.../libvxm_q8_trace.so) writes,
for every decode launch, trace_L<layers>_<n>.bin into $VXM_TRACE_DIR: for each of the 256 workgroups a row
of 2 + 16 * layers 64-bit values of the 100 MHz real-time counter -- [0] the workgroup's start, and per layer
l at 2 + 16 l + k:
  k = 0  layer input x read (phase A may start)     k = 1  A's QKV rows computed
  k = 3  attention inputs read (attention workgroups) k = 4 attention output published
  k = 2  scores computed (attention workgroups)      k = 11 softmax done, P.V starts
  k = 12 A's input normalised and quantized         k = 13 D's input normalised and quantized
  k = 15 E's second refills issued                  k = 14 E's input quantized
  k = 5  attention output read (C may start)        k = 6  C's O rows computed
  k = 7  h1 read (D may start)                      k = 8  D's gate / up rows computed
  k = 9  p read (E may start)                       k = 10 E's down rows computed
Row 0, value [1], is workgroup 0's start of the final RMSNorm.

Usage: python trace_phases.py <trace dir> [--skip N]   (N leading launches skipped, default 4: warm-up)
Prints a markdown table: per phase and per exchange ("hop": the previous phase's end in this workgroup to
this phase's inputs in it), the median and 90th percentile over workgroups and layers, in microseconds.
"""
import glob
import os
import sys

import numpy as np

TICK_US = 0.01   # 100 MHz
SLOTS = 16       # timestamps per layer


def load(path, n_wg=256):
    a = np.fromfile(path, dtype=np.uint64)
    stride = a.size // n_wg
    return a.reshape(n_wg, stride).astype(np.int64), (stride - 2) // SLOTS


def phases(t, L):
    """Durations in ticks: dict name -> array over (workgroups, layers) (NaN where not applicable)."""
    s = lambda k: t[:, 2 + np.arange(L) * SLOTS + k].astype(np.float64)
    att = s(3) > 0
    nan = np.full_like(s(0), np.nan)
    out = {
        "A: norm + QKV rows": s(1) - s(0),
        "  A norm + Q8_0": s(12) - s(0),
        "  QKV units": s(1) - s(12),
        "hop A -> attention inputs": np.where(att, s(3) - s(1), nan),
        "attention (incl. chunk merge)": np.where(att, s(4) - s(3), nan),
        "  scores (K rows landed + q.k)": np.where(att, s(2) - s(3), nan),
        "  softmax": np.where(att, s(11) - s(2), nan),
        "  P.V + reduction + Q8_0 + publish": np.where(att, s(4) - s(11), nan),
        "hop attention -> C inputs": np.where(att, s(5) - s(4), nan),
        "A end -> C inputs (every workgroup)": s(5) - s(1),
        "C: O rows + residual": s(6) - s(5),
        "hop C -> D inputs": s(7) - s(6),
        "D: norm + gate/up + SwiGLU": s(8) - s(7),
        "  D norm + Q8_0": s(13) - s(7),
        "  gate/up units": s(8) - s(13),
        "hop D -> E inputs": s(9) - s(8),
        "E: quant + down + residual": s(10) - s(9),
        "  refill issue": s(15) - s(9),
        "  Q8_0 of p": s(14) - s(15),
        "  down units": s(10) - s(14),
    }
    nxt = np.concatenate([s(0)[:, 1:], np.full((t.shape[0], 1), np.nan)], axis=1)
    out["hop E -> next layer's A inputs"] = nxt - s(10)
    out["layer (A inputs to next A inputs)"] = nxt - s(0)
    return out


def exchanges(t, L):
    """Per exchange and layer, in ticks: the spread of the producers' finish (last minus median
    workgroup), and the time from the LAST producer's finish to the median consumer having every
    input (the transit seen by the critical path)."""
    s = lambda k: t[:, 2 + np.arange(L) * SLOTS + k].astype(np.float64)
    att = s(3) > 0
    ends_next = [("A -> attention", s(1), np.where(att, s(3), np.nan)),
                 ("attention -> C", np.where(att, s(4), np.nan), s(5)),
                 ("C -> D", s(6), s(7)),
                 ("D -> E", s(8), s(9)),
                 ("E -> next A", s(10)[:, :-1], s(0)[:, 1:])]
    out = {}
    for name, end, ready in ends_next:
        last = np.nanmax(end, axis=0)
        out[name] = (last - np.nanmedian(end, axis=0), np.nanmedian(ready, axis=0) - last)
    return out


def main(argv):
    d = argv[1]
    skip = int(argv[argv.index("--skip") + 1]) if "--skip" in argv else 4
    files = sorted(glob.glob(os.path.join(d, "trace_L*_*.bin")))[skip:]
    if not files:
        raise SystemExit(f"no traces in {d}")
    acc = {}
    totals = []
    for f in files:
        t, L = load(f)
        for k, v in phases(t, L).items():
            acc.setdefault(k, []).append(v[np.isfinite(v)])
        end = t[0, 1]
        totals.append((end - t[:, 0].min()) * TICK_US)
    print(f"{len(files)} launches, {L} layers; launch start to final norm: median {np.median(totals):.1f} us")
    print()
    print("| step | median us | p90 us |")
    print("|---|---|---|")
    for k, parts in acc.items():
        v = np.concatenate(parts) * TICK_US
        print(f"| {k} | {np.median(v):.2f} | {np.percentile(v, 90):.2f} |")
    ex = {}
    for f in files:
        t, L = load(f)
        for k, (skew, transit) in exchanges(t, L).items():
            ex.setdefault(k, ([], []))
            ex[k][0].append(skew)
            ex[k][1].append(transit)
    print()
    print("| exchange | producers' finish: last - median, us | last producer -> median consumer ready, us |")
    print("|---|---|---|")
    for k, (skew, transit) in ex.items():
        print(f"| {k} | {np.median(np.concatenate(skew)) * TICK_US:.2f} | "
              f"{np.median(np.concatenate(transit)) * TICK_US:.2f} |")


if __name__ == "__main__":
    main(sys.argv)
