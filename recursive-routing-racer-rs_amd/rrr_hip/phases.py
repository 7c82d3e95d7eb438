"""Phase timestamps of the decode-path batch-1 GEMVs (rrr_probe_gemv_phases).

    python -m rrr_hip.phases [--launches 40] [--resident-x]

For each of the decode token's GEMV launches (RMSNorm + QKV Q5_K 5120x3072,
GQA-V + O-proj Q4_K 3072x3072 + residual, RMSNorm + gate/up Q4_K 16384x3072
with silu * up, down Q6_K / Q4_K 3072x8192 + residual) and the single Q4_K
3072x3072 GEMV, the stamped twin of the kernel runs `--launches` times over
rotating weight copies (over 600 MB a pass, so the weights stream from HBM),
each launch right after a kernel that writes its activation vector (as in
the decode token, where the previous op writes it), or with --resident-x
after a kernel that writes another buffer, so the activation vector stays
as the previous launch left it (as in the per-kernel bench lines).  Per
phase it prints the
median over launches of the median, 90th percentile and maximum over the
launch's waves of the phase's time after the launch's first wave started, in
microseconds (the device's 100 MHz constant clock), as a markdown table.
"""
import argparse
import sys

import numpy as np

from . import engine as E
from . import synth
from .engine import Context

PHASES = ["start", "activations landed", "after the RMSNorm scale", "activations encoded",
          "tile 0 block 0 staged", "tile 0 block 0 multiplied", "tile 0 block 1 staged", "tile 0 block 1 multiplied",
          "last tile block 0 staged", "last tile block 0 multiplied", "last tile block 1 staged",
          "last tile block 1 multiplied", "row partials written", "past the final barrier", "end (stores complete)"]

# name, op, weight type, K, N (F for the pair form), activation floats, act kind / param
CASES = [
    ("QKV: RMSNorm + Q5_K 5120x3072", E.PHASES_RMSNORM, E.Q5_K, 3072, 5120, 3072, 0, 0),
    ("O-proj: GQA-V + Q4_K 3072x3072 + residual", E.PHASES_RESIDUAL, E.Q4_K, 3072, 3072, 5120, E.ACT_GQA_V,
     128 | (3 << 16)),
    ("gate/up: RMSNorm + Q4_K 16384x3072, silu * up", E.PHASES_RMSNORM_SILU, E.Q4_K, 3072, 8192, 3072, 0, 0),
    ("down: Q6_K 3072x8192 + residual", E.PHASES_RESIDUAL, E.Q6_K, 8192, 3072, 8192, E.ACT_IDENTITY, 0),
    ("down: Q4_K 3072x8192 + residual", E.PHASES_RESIDUAL, E.Q4_K, 8192, 3072, 8192, E.ACT_IDENTITY, 0),
    ("single Q4_K 3072x3072", E.PHASES_PLAIN, E.Q4_K, 3072, 3072, 3072, 0, 0),
]


def measure(ctx, case, launches, warm=8, resident_x=False):
    name, op, qt, K, N, xlen, act_kind, act_param = case
    rows = 2 * N if op == E.PHASES_RMSNORM_SILU else N
    wbytes = E.tensor_bytes(qt, K, rows)
    copies = max(8, (640 << 20) // wbytes)
    Ws = [ctx.weight_upload(qt, K, rows, synth.weight(7, c, qt, K, rows)) for c in range(copies)]
    src = ctx.to_device(synth.normal_f32(7, 1, xlen))
    zero = ctx.to_device(np.zeros(xlen, np.float32))
    x = ctx.alloc(xlen * 4)
    gamma = ctx.to_device(synth.normal_f32(7, 2, K, 1.0, 0.1))
    y = ctx.to_device(synth.normal_f32(7, 3, N))
    cus = ctx.probe_cus()
    per = cus * 16 * 16 * 8
    st = ctx.alloc(per)
    ts = []
    grid = waves = 0
    other = ctx.alloc(xlen * 4)
    ctx.residual_add(src, zero, x, xlen)
    for r in range(warm + launches):
        # the previous kernel writes the activations, or (resident) another buffer
        ctx.residual_add(src, zero, other if resident_x else x, xlen)
        grid, waves = ctx.probe_gemv_phases(op, x, Ws[r % copies], qt, y, K, N, st, gamma=gamma,
                                            act_kind=act_kind, act_param=act_param)
        ctx.sync()
        if r >= warm:
            ts.append(ctx.download(st, np.uint64, grid * waves * 16).reshape(grid * waves, 16).astype(np.int64))
    for b in Ws + [src, zero, x, other, gamma, y, st]:
        b.free()
    stats = {}
    for k in range(len(PHASES)):
        rows_k = []
        for t in ts:
            v = t[:, k]
            v = v[v > 0]
            if v.size:
                d = (v - t[:, 0].min()) * 0.01
                rows_k.append((np.median(d), np.percentile(d, 90), d.max()))
        if rows_k:
            stats[k] = np.median(np.array(rows_k), axis=0)
    return wbytes, grid, waves, stats


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--launches", type=int, default=40)
    ap.add_argument("--resident-x", action="store_true",
                    help="no kernel writes the activations between launches")
    args = ap.parse_args(argv)
    with Context(0) as ctx:
        for case in CASES:
            wbytes, grid, waves, st = measure(ctx, case, args.launches, resident_x=args.resident_x)
            print(f"\n### {case[0]} ({wbytes / 1e6:.1f} MB of weights; {grid} workgroups of {waves} waves)\n")
            print("| phase | median us | p90 us | max us |")
            print("|---|---|---|---|")
            for k, (med, p90, mx) in sorted(st.items()):
                print(f"| {PHASES[k]} | {med:.2f} | {p90:.2f} | {mx:.2f} |")
            sys.stdout.flush()


if __name__ == "__main__":
    main()
