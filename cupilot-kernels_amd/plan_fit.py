"""Fit the constants of the planner's dense cost model (csrc/scheduler.cpp,
kModels and the reduction / stream-K constants) to measured plan timings.

The model is the one plan_gemm evaluates (batch and layout from the table;
operands contiguous, so a row's leading dimensions are its extents):
  per_cu = ceil(items / CUs), occ = min(resident workgroups, per_cu)
  t      = per_cu * 2 BM BN kc / (eff[cfg][occ] * CU peak) + ceil(items / grid) * item_ns[cfg]
           + store_exp[cfg][occ > 1] * out_bytes * split / write bandwidth
           + (split > 1) * ((split + 1) * out_bytes / reduce bandwidth + reduce_ns)
  stream-K: the work spread over every resident workgroup, (dp / G + 2) items,
           partial tiles stored and read back three times, sk_slot_ns * G / S; on the
           k-split 64 tile its own efficiency factor and fixed cost (sk10_eff, sk10_ns).
  Operands the 16-byte loaders cannot stage (a row or K not a multiple of 4 floats,
  or K off the tile's slice depth) scale the efficiency: the 128 tile's 4-byte
  direct staging by e2v (data-parallel and split-K, plus o2v per work item) and
  sk2v (stream-K, plus sk2v_ns per work item), the register-staged 64 and 256 tiles by s1v and s3v;
  with C rows not 16-byte aligned the reduction and fixup passes, which then
  run element-wise, reach rv of their bandwidth, and the output stores (also
  element-wise) take xv times as long.
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
BM = {1: 64, 2: 128, 3: 256, 9: 128, 10: 64, 11: 128}
BK = {1: 16, 2: 16, 3: 32, 9: 32, 10: 64, 11: 32}
RES = {1: 8, 2: 3, 3: 1, 9: 2, 10: 1, 11: 2}
NAMES = ["e1_1", "e1_2", "e1_3", "e2_1", "e2_2", "e2_3", "e3", "e9_1", "e9_2",
         "o1", "o2", "o3", "o9", "x3", "x_occ1", "x_occ2", "reduce_bw", "reduce_ns", "sk_slot_ns",
         "e10", "o10", "x10", "sk10_eff", "sk10_ns", "s1v", "s3v", "e2v", "sk2v", "sk2v_ns", "rv", "xv", "o2v", "e11_1", "e11_2", "o11"]
# the constants csrc/scheduler.cpp carries (the starting point of the search)
X0 = [0.4263, 0.654, 0.72, 0.8892, 0.91, 0.9178, 0.9547, 0.861, 0.9231, 2961, 2904, 1.372, 4510, 1.447, 1.5, 0.4952, 7592, 5354, 962.3, 0.85, 2361, 0.733, 0.798, 0, 0.5706, 0.8389, 0.8815, 1.121, 5552, 0.2811, 5.497, 1010, 0.995, 0.9354, 4815]
LO = [0.2] * 9 + [0.0] * 4 + [0.0, 0.0, 0.0, 1000, 0, 0] + [0.2, 0.0, 0.0, 0.3, 0.0] + [0.2] * 4 + [0.0, 0.05, 0.5, 0.0] + [0.2, 0.2, 0.0]
HI = [1.2] * 9 + [5e4] * 4 + [1.5, 1.5, 1.5, 2e4, 5e4, 5e4] + [1.2, 5e4, 1.5, 1.2, 5e4] + [1.2, 1.2, 1.2, 1.5] + [5e4, 1.5, 12.0, 5e4] + [1.2, 1.2, 5e4]


PINNED = {(8192, 8192, 8192, 1, "NN"), (8192, 8192, 8192, 1, "TN"), (8192, 8192, 8192, 1, "NT"),
          (8192, 8192, 8192, 1, "TT"), (512, 768, 1024, 128, "NN"), (16384, 768, 2048, 1, "NN"),
          (65536, 512, 256, 1, "NN"), (1024, 1024, 1024, 1, "NN"), (2048, 4096, 8192, 1, "NN"),
          (2048, 8192, 4096, 1, "NN"), (3072, 3072, 8192, 1, "NN"), (4608, 4608, 4608, 1, "NN"),
          (4096, 4096, 512, 1, "NN"),
          (8205, 5921, 2976, 1, "NT")}  # (the last: PID 8's product after packing)


def cdiv(a, b):
    return -(-a // b)


def vec4(r):
    """16-byte operand rows (choose_vec == 4) for contiguous operands."""
    M, N, K, lay = r["M"], r["N"], r["K"], r["layout"]
    return ((K if lay[0] == "N" else M) % 4 == 0) and ((N if lay[1] == "N" else K) % 4 == 0)


def sk4_allowed(M, N, K):
    """The planner's guard on stream-K with 4-byte staging (scheduler.cpp,
    plan_stream_k): K >= 1536, at least G / 6 tiles, and a data-parallel plan
    whose per-CU tile count is >= 12 % above the mean."""
    T, G = cdiv(M, 128) * cdiv(N, 128), NC * RES[2]
    return K >= 1536 and 6 * T >= G and cdiv(T, NC) * NC >= 1.12 * T


def model(r, x):
    P = dict(zip(NAMES, x))
    M, N, K, B, c, s, sk = r["M"], r["N"], r["K"], r["batch"], r["cfg"], r["split"], r["stream_k"]
    bm = BM[c]
    T = cdiv(M, bm) * cdiv(N, bm) * B
    out = 4.0 * M * N * B
    v4 = vec4(r)
    # C rows not 16-byte aligned: the split-K reduction and the stream-K fixup
    # run element-wise (bandwidth factor rv)
    red = 1.0 if N % 4 == 0 else 1.0 / P["rv"]
    xst = 1.0 if N % 4 == 0 else P["xv"]  # (and the output stores are element-wise)
    four_byte = c == 2 and not (v4 and K % 16 == 0)
    scale = (P["s3v"] if c == 3 and not (v4 and K % 32 == 0) else P["s1v"] if c == 1 and not v4
             else P["e2v"] if four_byte and not sk else 1.0)
    eff = {1: [P["e1_1"], P["e1_2"], P["e1_3"]], 2: [P["e2_1"], P["e2_2"], P["e2_3"]],
           3: [P["e3"]] * 3, 9: [P["e9_1"], P["e9_2"], P["e9_2"]], 10: [P["e10"]] * 3,
           11: [P["e11_1"], P["e11_2"], P["e11_2"]]}[c]
    xs = ([P["x3"], P["x3"]] if c == 3 else [P["x10"], P["x10"]] if c == 10
          else [P["x_occ1"], P["x_occ2"]])
    o = P["o%d" % c]
    if sk and four_byte and not sk4_allowed(M, N, K):
        return math.inf  # the planner does not offer it
    if sk:
        G = NC * RES[c]
        waves = T // G
        dp = (waves - 1) * G if waves >= 1 else 0
        S = T - dp
        tile = 4.0 * bm * bm
        ske = P["sk10_eff"] if c == 10 else P["sk2v"] if four_byte else 1.0
        t = T * 2.0 * bm * bm * K / NC / (scale * ske * eff[min(RES[c], 3) - 1] * PEAK)
        t += P["sk10_ns"] if c == 10 else 0.0
        t += (dp // G + 2) * (o + (P["sk2v_ns"] if four_byte else 0.0))
        t += xs[1 if RES[c] > 1 else 0] * (xst * out + G * tile) / WRITE
        t += 3.0 * G * tile / P["reduce_bw"] * red + P["sk_slot_ns"] * G / S
        return t
    items = T * s
    kc = cdiv(cdiv(K, s), BK[c]) * BK[c]
    per_cu = cdiv(items, NC)
    occ = min(RES[c], per_cu)
    grid = min(NC * RES[c], items)
    # full rounds of RES[c] resident tiles at that occupancy, then the tail's
    # leftover tiles at their own (lower) occupancy
    rounds, rem = divmod(per_cu, occ)
    slots = rounds * occ / eff[min(occ, 3) - 1] + (rem / eff[min(rem, 3) - 1] if rem else 0.0)
    t = (slots * 2.0 * bm * bm * kc / (scale * PEAK)
         + cdiv(items, grid) * (o + (P["o2v"] if four_byte else 0.0)))
    t += xs[1 if occ > 1 else 0] * xst * out * s / WRITE
    if s > 1:
        t += (s + 1) * out / P["reduce_bw"] * red + P["reduce_ns"]
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
    ap.add_argument("--only", default="", help="comma-separated constants to search (default: all)")
    args = ap.parse_args(argv)
    free = [NAMES.index(n) for n in args.only.split(",") if n] or list(range(len(NAMES)))
    rows = [r for r in load(args.table) if r["cfg"] in BM]
    by = defaultdict(list)
    for r in rows:
        by[(r["M"], r["N"], r["K"], r["batch"], r["layout"])].append(r)
    best = {k: min(r["ms"] for r in v) for k, v in by.items()}
    key = lambda r: (r["M"], r["N"], r["K"], r["batch"], r["layout"])  # noqa: E731
    w = np.array([1.0 if r["ms"] <= 1.15 * best[key(r)] else 0.25 for r in rows])

    def resid(x):
        return w * np.array([math.log(model(r, x) / (r["ms"] * 1e6)) if math.isfinite(model(r, x)) else 0.0
                             for r in rows])

    def pick(v, x):
        # plan_gemm's order (kModels: 256, 128, 64, ..., then split 1, 2, 4, ...
        # before stream-K per config) and its rule: a later plan replaces the
        # best so far only if at least 0.1 % faster
        order = {3: 0, 2: 1, 1: 2, 9: 5, 10: 6, 11: 7}
        best_r, best_t = None, math.inf
        for r in sorted(v, key=lambda r: (order[r["cfg"]], r["stream_k"], r["split"])):
            if r["cfg"] == 11 and (r["split"] > 1 or r["stream_k"] or r["K"] < 1024):
                continue  # the planner offers the 8-wave tile data-parallel from K = 1024
            if r["stream_k"] and r["K"] < 1024:
                continue  # nor stream-K below K = 1024
            t = model(r, x)
            if t < best_t * 0.999:
                best_r, best_t = r, t
        return best_r

    def regrets(x):
        return [pick(v, x)["ms"] / best[k] - 1 for k, v in by.items()]

    # the BASELINE configs' shapes (and PID 2's): the planner must stay within
    # 1 % of their best measured plan (tests/test_abi_cpu.py holds it to that);
    # 4096^2 x 512 likewise (the shallow-K shape the tests expect on the 128
    # tile, where the model has the 256 tile within a hair of it)
    pinned = [k for k in by if k in PINNED]

    def score(x):
        reg = regrets(x)
        pin = sum(max(0.0, pick(by[k], x)["ms"] / best[k] - 1.01) for k in pinned)
        return np.mean(reg) + 0.1 * max(reg) + 0.2 * float(np.sqrt(np.mean(resid(x) ** 2))) + 10.0 * pin

    def report(x, what):
        reg = regrets(x)
        print(f"{what}: rms log error {np.sqrt(np.mean((resid(x) / w) ** 2)):.3f}; regret of the picked plan: "
              f"mean {np.mean(reg) * 100:.2f} %, max {max(reg) * 100:.1f} %")
        for name, sel in (("16-byte rows", True), ("4-byte rows", False)):
            sub = [g for g, k in zip(reg, by) if vec4(by[k][0]) == sel]
            if sub:
                print(f"  {name}: {len(sub)} shapes, mean {np.mean(sub) * 100:.2f} %, max {max(sub) * 100:.1f} %")

    print(f"{len(rows)} timings, {len(by)} shapes")
    report(np.array(X0), "scheduler.cpp constants")
    x = least_squares(resid, X0, bounds=(LO, HI)).x if args.lsq else np.array(X0, dtype=float)
    rng = np.random.default_rng(0)
    cur, cs = np.array(x), score(x)
    lo, hi = np.array(LO), np.array(HI)
    for _ in range(args.iters):
        cand = cur.copy()
        k = rng.choice(free, size=min(len(free), int(rng.integers(1, 4))), replace=False)
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
