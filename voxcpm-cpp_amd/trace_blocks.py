"""Per-phase timeline of k_locdit_persistent from the profiling build's timestamps.

Usage: python3 trace_blocks.py <dir with ltrace_L*_M*_*.bin> [rows M] [launches to skip] [blocks per evaluation]

Every workgroup writes the 100 MHz real-time counter at its start and, per
block, at 24 points: 0 block start; then for each phase (N1, QKV, ATT, O, N2,
GU, D) the moment its inputs are in LDS (odd slots 1..13, written only by the
workgroups that have that phase) and the moment the workgroup leaves the phase
(even slots 2..14); slot 15 = the last block's final inputs; 16..23 steps inside
QKV (products, partial sums), the attention (scores, softmax, P.V) and gate/up
(products, partial sums, SwiGLU); in a CFM solve traced as one launch (its blocks
numbered over the evaluations), 24 / 25 the row owners' assembly of an evaluation's
rows (inputs in LDS, done) at its first block and 26 / 27 the update workgroup's
out_proj + Euler step (inputs, done) at its last block, 28-31 inside that step (products,
out_proj rows, CFG sums, Euler step + Q8_0), slot 15 there the x rows' owners holding the
last down partials.  For each phase:
  hop   = from the last producer leaving the previous phase to the median
          consumer having all its inputs,
  work  = from the median consumer's inputs to the last consumer leaving.
"""
import glob
import os
import sys

import numpy as np

SLOTS = 32
PHASES = ["N1 (norm)", "QKV", "attention", "O", "N2 (norm)", "gate/up", "down"]


def load(path):
    base = os.path.basename(path)
    L = int(base.split("_L")[1].split("_")[0])
    a = np.fromfile(path, dtype=np.uint64).astype(np.int64)
    return L, a.reshape(256, 1 + SLOTS * L)


def main():
    d = sys.argv[1]
    rows = sys.argv[2] if len(sys.argv) > 2 else "*"
    skip = int(sys.argv[3]) if len(sys.argv) > 3 else 1
    files = sorted(glob.glob(os.path.join(d, f"ltrace_L*_M{rows}_*.bin")))[skip:]
    if not files:
        sys.exit("no ltrace files")
    rows = {p: ([], []) for p in PHASES}
    totals = []
    for f in files:
        L, t = load(f)
        start = t[:, 0]
        totals.append((t[:, 1 + SLOTS * (L - 1) + 14].max() - start.min()) / 100.0)
        for l in range(L):
            m = t[:, 1 + SLOTS * l: 1 + SLOTS * (l + 1)]
            prev_done = None if l == 0 else t[:, 1 + SLOTS * (l - 1) + 14]
            for k, name in enumerate(PHASES):
                ready, done = m[:, 2 * k + 1], m[:, 2 * k + 2]
                who = ready > 0
                if not who.any():
                    continue
                if k == 0:
                    if prev_done is None:
                        continue
                    last_prod = prev_done.max()
                else:
                    pr = m[:, 2 * k - 1] > 0
                    last_prod = m[pr, 2 * k].max()
                hop = (np.median(ready[who]) - last_prod) / 100.0
                work = (done[who].max() - np.median(ready[who])) / 100.0
                rows[name][0].append(hop)
                rows[name][1].append(work)
    print(f"{len(files)} launches; launch start to last block's down: median {np.median(totals):.1f} us")
    print("| phase | hop us (median) | work us (median) |")
    print("|---|---|---|")
    th = tw = 0.0
    for name in PHASES:
        h, w = rows[name]
        if not h:
            continue
        th += np.median(h)
        tw += np.median(w)
        print(f"| {name} | {np.median(h):.2f} | {np.median(w):.2f} |")
    print(f"| per block | {th:.2f} | {tw:.2f} |")
    # steps inside phases: median over the workgroups that run them of (slot b - slot a)
    steps = [("QKV: products", 3, 16), ("QKV: partial sums to LDS", 16, 17), ("QKV: epilogue + publish", 17, 4),
             ("attention: scores", 5, 22), ("attention: softmax", 22, 23), ("attention: P.V", 23, 21),
             ("attention: Q8_0 + publish", 21, 6),
             ("gate/up: products", 11, 18), ("gate/up: partial sums to LDS", 18, 19), ("gate/up: SwiGLU", 19, 20),
             ("gate/up: Q8_0 + publish", 20, 12)]
    sub = {n: [] for n, _, _ in steps}
    for f in files:
        L, t = load(f)
        for l in range(L):
            m = t[:, 1 + SLOTS * l: 1 + SLOTS * (l + 1)]
            for n, a, b in steps:
                w = (m[:, a] > 0) & (m[:, b] > 0)
                if w.any():
                    sub[n].append(np.median(m[w, b] - m[w, a]) / 100.0)
    print()
    print("| step inside a phase (one workgroup) | median us |")
    print("|---|---|")
    for n, _, _ in steps:
        if sub[n]:
            print(f"| {n} | {np.median(sub[n]):.2f} |")
    # a solve: the exchanges between two evaluations, from the last down products of
    # evaluation k - 1 to the first N1 inputs of evaluation k
    per = int(sys.argv[4]) if len(sys.argv) > 4 else 0
    if per:
        tail = {n: [] for n in ("down done -> x rows' partials in LDS", "-> update inputs in LDS", "update work",
                                "-> x rows' assembly inputs in LDS", "x rows' assembly work",
                                "-> every row's N1 done", "between evaluations (down done -> N1 done)")}
        for f in files:
            L, t = load(f)
            for k in range(1, L // per):
                a = t[:, 1 + SLOTS * (k * per - 1): 1 + SLOTS * k * per]
                b = t[:, 1 + SLOTS * k * per: 1 + SLOTS * (k * per + 1)]
                d_done = a[:, 14].max()
                xr = a[:, 15] > 0          # the x rows' owners
                upd = a[:, 26] > 0
                own = b[:, 2] > 0          # every row owner's N1
                if not (xr.any() and upd.any() and own.any()):
                    continue
                u_in, u_done = a[upd, 26].max(), a[upd, 27].max()
                tail["down done -> x rows' partials in LDS"].append((np.median(a[xr, 15]) - d_done) / 100.0)
                tail["-> update inputs in LDS"].append((u_in - np.median(a[xr, 15])) / 100.0)
                tail["update work"].append((u_done - u_in) / 100.0)
                prev = u_in
                for sl, nm in ((28, "  out_proj products"), (29, "  out_proj rows"), (30, "  CFG sums"),
                               (31, "  Euler step + Q8_0"), (27, "  publish")):
                    tail.setdefault(nm, []).append((a[upd, sl].max() - prev) / 100.0)
                    prev = a[upd, sl].max()
                tail["-> x rows' assembly inputs in LDS"].append((np.median(b[xr, 24]) - u_done) / 100.0)
                tail["x rows' assembly work"].append((b[xr, 25].max() - np.median(b[xr, 24])) / 100.0)
                tail["-> every row's N1 done"].append((b[own, 2].max() - b[xr, 25].max()) / 100.0)
                tail["between evaluations (down done -> N1 done)"].append((b[own, 2].max() - d_done) / 100.0)
        print()
        print("| between two evaluations of a solve | median us |")
        print("|---|---|")
        for n, v in tail.items():
            if v:
                print(f"| {n} | {np.median(v):.2f} |")


if __name__ == "__main__":
    main()
