"""Fit the constants of the planner's dense cost model (csrc/scheduler.cpp,
kModels and the reduction / stream-K constants) to measured plan timings.

The model is the one plan_gemm evaluates (N/N, 16-byte operands, batch from
the table):
  per_cu = ceil(items / CUs), occ = min(resident workgroups, per_cu)
  t      = per_cu * 2 BM BN kc / (eff[cfg][occ] * CU peak) + ceil(items / grid) * item_ns[cfg]
           + store_exp[cfg][occ > 1] * out_bytes * split / write bandwidth
           + (split > 1) * ((split + 1) * out_bytes / reduce bandwidth + reduce_ns)
  stream-K: the work spread over every resident workgroup, (dp / G + 2) items,
           partial tiles stored and read back three times, sk_slot_ns * G / S; on the
           k-split 64 tile its own efficiency factor and fixed cost (sk10_eff, sk10_ns).
Fit: a random local search on the ranking (mean regret of the plan the model
picks + 0.1 x worst regret + 0.2 x rms log error, plans within 15 % of a
shape's best weighing 4x in the rms) from the constants scheduler.cpp
carries; --lsq starts it from a least-squares fit on log time instead.
Prints the score of the starting constants and the constants it ends at.

usage: python cupilot-kernels_amd/plan_fit.py tests/data/plan_timings_mi355x.csv [--iters 2500] [--lsq]
"""
from __future__ import annotations

import argparse
import csv
import math
from collections import defaultdict

import numpy as np
from scipy.optimize import least_squares

NC = 256
PEAK = 256 * 2.4  # fp32 MFMA flop per ns per CU
WRITE = 5500.0
BM = {1: 64, 2: 128, 3: 256, 9: 128, 10: 64}
BK = {1: 16, 2: 16, 3: 32, 9: 32, 10: 64}
RES = {1: 8, 2: 3, 3: 1, 9: 2, 10: 1}
NAMES = ["e1_1", "e1_2", "e1_3", "e2_1", "e2_2", "e2_3", "e3", "e9_1", "e9_2",
         "o1", "o2", "o3", "o9", "x3", "x_occ1", "x_occ2", "reduce_bw", "reduce_ns", "sk_slot_ns",
         "e10", "o10", "x10", "sk10_eff", "sk10_ns"]
# the constants csrc/scheduler.cpp carries (the starting point of the search)
X0 = [0.433, 0.642, 0.718, 0.821, 0.907, 0.915, 0.947, 0.850, 0.914, 2937, 3393, 220, 4286, 1.38, 0.935,
      0.495, 7661, 5354, 930, 0.850, 2361, 0.733, 0.798, 0.0]
LO = [0.2] * 9 + [0.0] * 4 + [0.0, 0.0, 0.0, 1000, 0, 0] + [0.2, 0.0, 0.0, 0.3, 0.0]
HI = [1.2] * 9 + [5e4] * 4 + [1.5, 1.5, 1.5, 2e4, 5e4, 5e4] + [1.2, 5e4, 1.5, 1.2, 5e4]


def cdiv(a, b):
    return -(-a // b)


def model(r, x):
    P = dict(zip(NAMES, x))
    M, N, K, B, c, s, sk = r["M"], r["N"], r["K"], r["batch"], r["cfg"], r["split"], r["stream_k"]
    bm = BM[c]
    T = cdiv(M, bm) * cdiv(N, bm) * B
    out = 4.0 * M * N * B
    scale = 0.75 if (c == 3 and K % 32) else 1.0
    eff = {1: [P["e1_1"], P["e1_2"], P["e1_3"]], 2: [P["e2_1"], P["e2_2"], P["e2_3"]],
           3: [P["e3"]] * 3, 9: [P["e9_1"], P["e9_2"], P["e9_2"]], 10: [P["e10"]] * 3}[c]
    xs = ([P["x3"], P["x3"]] if c == 3 else [P["x10"], P["x10"]] if c == 10
          else [P["x_occ1"], P["x_occ2"]])
    o = P["o%d" % c]
    if sk:
        G = NC * RES[c]
        waves = T // G
        dp = (waves - 1) * G if waves >= 1 else 0
        S = T - dp
        tile = 4.0 * bm * bm
        ske = P["sk10_eff"] if c == 10 else 1.0
        t = T * 2.0 * bm * bm * K / NC / (scale * ske * eff[min(RES[c], 3) - 1] * PEAK)
        t += P["sk10_ns"] if c == 10 else 0.0
        t += (dp // G + 2) * o
        t += xs[1 if RES[c] > 1 else 0] * (out + G * tile) / WRITE
        t += 3.0 * G * tile / P["reduce_bw"] + P["sk_slot_ns"] * G / S
        return t
    items = T * s
    kc = cdiv(cdiv(K, s), BK[c]) * BK[c]
    per_cu = cdiv(items, NC)
    occ = min(RES[c], per_cu)
    grid = min(NC * RES[c], items)
    t = per_cu * 2.0 * bm * bm * kc / (scale * eff[min(occ, 3) - 1] * PEAK) + cdiv(items, grid) * o
    t += xs[1 if occ > 1 else 0] * out * s / WRITE
    if s > 1:
        t += (s + 1) * out / P["reduce_bw"] + P["reduce_ns"]
    return t


def load(path):
    rows = []
    with open(path) as f:
        for r in csv.DictReader(line for line in f if not line.startswith("#")):
            rows.append({k: (v if k == "layout" else (float(v) if k == "ms" else int(v))) for k, v in r.items()})
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("table")
    ap.add_argument("--iters", type=int, default=2500)
    ap.add_argument("--lsq", action="store_true")
    args = ap.parse_args(argv)
    rows = [r for r in load(args.table) if r["cfg"] in BM]
    by = defaultdict(list)
    for r in rows:
        by[(r["M"], r["N"], r["K"], r["batch"], r["layout"])].append(r)
    best = {k: min(r["ms"] for r in v) for k, v in by.items()}
    key = lambda r: (r["M"], r["N"], r["K"], r["batch"], r["layout"])  # noqa: E731
    w = np.array([1.0 if r["ms"] <= 1.15 * best[key(r)] else 0.25 for r in rows])

    def resid(x):
        return w * np.array([math.log(model(r, x) / (r["ms"] * 1e6)) for r in rows])

    def regrets(x):
        return [min(v, key=lambda r: model(r, x))["ms"] / best[k] - 1 for k, v in by.items()]

    def score(x):
        reg = regrets(x)
        return np.mean(reg) + 0.1 * max(reg) + 0.2 * float(np.sqrt(np.mean(resid(x) ** 2)))

    def report(x, what):
        reg = regrets(x)
        print(f"{what}: rms log error {np.sqrt(np.mean((resid(x) / w) ** 2)):.3f}; regret of the picked plan: "
              f"mean {np.mean(reg) * 100:.2f} %, max {max(reg) * 100:.1f} %")

    print(f"{len(rows)} timings, {len(by)} shapes")
    report(np.array(X0), "scheduler.cpp constants")
    x = least_squares(resid, X0, bounds=(LO, HI)).x if args.lsq else np.array(X0, dtype=float)
    rng = np.random.default_rng(0)
    cur, cs = np.array(x), score(x)
    lo, hi = np.array(LO), np.array(HI)
    for _ in range(args.iters):
        cand = cur.copy()
        k = rng.integers(len(cand), size=rng.integers(1, 4))
        cand[k] *= np.exp(rng.normal(0, 0.04, size=len(k)))
        cand = np.clip(cand, lo, hi)
        sc = score(cand)
        if sc < cs:
            cur, cs = cand, sc
    report(cur, "after the search")
    for n, v in zip(NAMES, cur):
        print(f"  {n} = {v:.4g}")


if __name__ == "__main__":
    main()
