"""Evaluation runner: every operator of this package against the PyTorch-ROCm
eager operator it replaces, on one MI355X, written in the schema of the
reference's results table (latency_summary.csv:1):

    Problem_ID,Kernels,Target_PyTorch_Latency(ms),Generated_Kernel_Latency(ms),Ratio_to_Target

``Target_PyTorch_Latency`` is the torch eager operator of the problem (the
KernelBench-style model body: ``A @ B``, ``torch.bmm``, ``torch.diag(a) @ B``,
``torch.tril(A @ B)``, ``F.conv2d`` ...) on the same GPU and inputs;
``Generated_Kernel_Latency`` is this package's operator; the ratio is
target / generated (> 1 = faster than torch), as in the reference table.  A
second, extended table adds the shape, the throughput, the result's
normalised difference from the torch result and, with ``--cpu``, the host CPU
time of the same torch operator.

    python cupilot-kernels_amd/evaluate.py --out gpurun_out/latency_summary_mi355x.csv
    python cupilot-kernels_amd/evaluate.py --preset small --pids 1,5,87 --out /tmp/t.csv

Shapes (``--preset baseline``) are BASELINE's configs where one names the
operator, else the reference's own literal extents (PID 2, kernels/2_...:16-18)
or a stated synthetic shape.  Inputs are uniform[-1, 1) from the library's
counter-based generator, resident in HBM before timing.  Both operators get
``--warmup`` untimed calls; then ``--rounds`` rounds alternate them, each
round timing ``--reps`` calls of one and then of the other between HIP events
on the current stream (the order flips every round, so neither always runs
first); a latency is the median over the rounds of the mean per call, output
allocation included (as KernelBench times a call).
With ``--cpu`` the host torch operator is timed on the same inputs (best of 3
calls after one warm-up call, all host threads) after every GPU timing.
"""
from __future__ import annotations

import argparse
import csv
import math
import os
import sys
import time
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence

HEADER = ["Problem_ID", "Kernels", "Target_PyTorch_Latency(ms)", "Generated_Kernel_Latency(ms)",
          "Ratio_to_Target"]
EXT_HEADER = HEADER + ["Shape", "Work", "Generated_Throughput", "Unit", "Max_Norm_Diff_vs_Torch",
                       "CPU_Torch_Latency(ms)", "CPU_Threads"]
KERNELS_LABEL = "mi355_gemm MI355X"


@dataclass
class Problem:
    pid: int
    shape: str
    make: Callable[[Callable], tuple]        # fill -> inputs
    ours: Callable[..., object]
    torch_ref: Callable[..., object]
    flops: float = 0.0                       # algorithmic work
    nbytes: float = 0.0                      # compulsory HBM bytes (bandwidth-bound problems)
    k_norm: int = 1                          # reduction length for the normalised difference
    note: str = ""
    extra: Dict[str, object] = field(default_factory=dict)


def _problems(ck, preset: str) -> List[Problem]:
    import torch
    import torch.nn.functional as F

    small = preset == "small"
    n8 = 256 if small else 8192
    P: List[Problem] = []

    def mm(pid, M, K, N, ta=False, tb=False, fn=None, ref=None, note=""):
        def make(u):
            a = u((K, M) if ta else (M, K), 16 * pid)
            b = u((N, K) if tb else (K, N), 16 * pid + 1)
            return a, b
        op_a = (lambda a: a.t()) if ta else (lambda a: a)
        op_b = (lambda b: b.t()) if tb else (lambda b: b)
        P.append(Problem(pid, f"{M}x{K}x{N}" + (" A^T" if ta else "") + (" B^T" if tb else ""), make,
                         fn, ref or (lambda a, b: op_a(a) @ op_b(b)), 2.0 * M * N * K, k_norm=K,
                         note=note))

    mm(1, n8, n8, n8, fn=ck.p01.matmul_cuda, note="BASELINE configs[1] NN")
    if small:
        mm(2, 128, 512, 256, fn=ck.p02.matmul_cuda)
    else:
        mm(2, 2048, 8192, 4096, fn=ck.p02.matmul_cuda, note="kernels/2_...:16-18 extents")

    b3 = (4, 64, 96, 80) if small else (128, 512, 1024, 768)
    P.append(Problem(3, "x".join(map(str, b3)),
                     lambda u: (u((b3[0], b3[1], b3[2]), 48), u((b3[0], b3[2], b3[3]), 49)),
                     ck.p03.batched_matmul_cuda, lambda a, b: torch.bmm(a, b),
                     2.0 * b3[0] * b3[1] * b3[2] * b3[3], k_norm=b3[2], note="BASELINE configs[2]"))

    gm, gk = (512, 4096) if small else (32768, 65536)
    P.append(Problem(4, f"{gm}x{gk}", lambda u: (u((gm, gk), 64), u((gk, 1), 66)),
                     ck.p04.gemv_cuda, lambda a, x: a @ x, 2.0 * gm * gk,
                     4.0 * (gm * gk + gk + gm), k_norm=gk, note="BASELINE configs[3]"))

    sm_, sn = (256, 512) if small else (16384, 4096)
    P.append(Problem(5, f"{sm_}x{sn}", lambda u: (u((sm_, sn), 80), 3.14),
                     ck.p05.matrix_scalar_mult_cuda, lambda a, s: a * s, 0.0,
                     8.0 * sm_ * sn, note="synthetic 256 MiB (no BASELINE config)"))

    lk = 1 << 14 if small else 1 << 20
    P.append(Problem(6, f"256x{lk}x256", lambda u: (u((256, lk), 96), u((lk, 256), 97)),
                     ck.p06.matmul_cuda, lambda a, b: a @ b, 2.0 * 256 * 256 * lk, k_norm=lk,
                     note="BASELINE configs[4]"))

    skm = 1024 if small else 16384
    P.append(Problem(7, f"{skm}x32x{skm}", lambda u: (u((skm, 32), 112), u((32, skm), 113)),
                     ck.p07.gemm_cuda, lambda a, b: a @ b, 2.0 * skm * skm * 32,
                     4.0 * (2 * skm * 32 + skm * skm), k_norm=32, note="BASELINE configs[3]"))

    if small:
        mm(8, 67, 129, 31, fn=ck.p08.matmul_cuda)
    else:
        mm(8, 8205, 2949, 5921, fn=ck.p08.matmul_cuda, note="synthetic irregular extents")

    tm = 2048 if small else 65536
    P.append(Problem(9, f"{tm}x64", lambda u: (u((tm, 64), 144), u((64, tm), 145)),
                     ck.p09.tall_skinny_matmul_cuda, lambda a, b: a @ b, 2.0 * tm * tm * 64,
                     4.0 * (2 * tm * 64 + tm * tm), k_norm=64, note="BASELINE configs[4]"))

    t3 = (2, 64, 128, 96) if small else (16, 1024, 2048, 768)
    P.append(Problem(10, "x".join(map(str, t3)),
                     lambda u: (u((t3[0], t3[1], t3[2]), 160), u((t3[2], t3[3]), 161)),
                     ck.p10.batched_matmul_cuda, lambda a, b: torch.matmul(a, b),
                     2.0 * t3[0] * t3[1] * t3[2] * t3[3], k_norm=t3[2], note="BASELINE configs[2]"))

    t4 = (2, 4, 8, 64, 32) if small else (8, 64, 128, 256, 512)
    P.append(Problem(11, "x".join(map(str, t4)),
                     lambda u: (u(t4[:4], 176), u((t4[3], t4[4]), 177)),
                     ck.p11.tensor_matmul_cuda, lambda a, b: torch.matmul(a, b),
                     2.0 * t4[0] * t4[1] * t4[2] * t4[3] * t4[4], k_norm=t4[3],
                     note="BASELINE configs[2]"))

    dn = 512 if small else 8192
    P.append(Problem(12, f"{dn}x{dn}", lambda u: (u((dn,), 192), u((dn, dn), 193)),
                     ck.p12.diag_mult_cuda, lambda a, b: torch.diag(a) @ b, 0.0,
                     4.0 * (dn + 2 * dn * dn), note="BASELINE configs[3]"))

    def sym(u):
        r1, r2 = u((n8, n8), 208), u((n8, n8), 209)
        return (r1 + r1.t()) / 2, (r2 + r2.t()) / 2
    P.append(Problem(13, f"{n8}", sym, ck.p13.symmetric_matmul_cuda, lambda a, b: a @ b,
                     2.0 * n8 ** 3, k_norm=n8, note="BASELINE configs[4]"))
    tri = n8 * (n8 + 1) * (n8 + 2) / 3.0
    P.append(Problem(14, f"{n8}", lambda u: (torch.triu(u((n8, n8), 224)), torch.triu(u((n8, n8), 225))),
                     ck.p14.upper_tri_matmul_cuda, lambda a, b: torch.triu(a @ b), tri, k_norm=n8,
                     note="BASELINE configs[4]"))
    P.append(Problem(15, f"{n8}", lambda u: (torch.tril(u((n8, n8), 240)), torch.tril(u((n8, n8), 241))),
                     ck.p15.lower_tri_mul_cuda, lambda a, b: torch.tril(a @ b), tri, k_norm=n8,
                     note="BASELINE configs[4]"))
    mm(16, n8, n8, n8, ta=True, fn=ck.p16.matmul_transposed_cuda, note="BASELINE configs[1] TN")
    mm(17, n8, n8, n8, tb=True, fn=ck.p17.matmul_cuda, note="BASELINE configs[1] NT")
    mm(18, n8, n8, n8, ta=True, tb=True, fn=ck.p18.matmul_transposed_cuda,
       note="BASELINE configs[1] TT")

    cv = (2, 16, 32, 32, 32) if small else (16, 64, 128, 256, 256)   # n, cin, cout, h, w
    P.append(Problem(87, "x".join(map(str, cv)),
                     lambda u: (u((cv[0], cv[1], cv[3], cv[4]), 1392), u((cv[2], cv[1], 1, 1), 1393),
                                u((cv[2],), 1394)),
                     ck.p87.pointwise_conv_cuda, lambda x, w, b: F.conv2d(x, w, b),
                     2.0 * cv[0] * cv[1] * cv[2] * cv[3] * cv[4],
                     4.0 * (cv[0] * cv[1] * cv[3] * cv[4] + cv[2] * cv[1] + cv[2]
                            + cv[0] * cv[2] * cv[3] * cv[4]),
                     k_norm=cv[1], note="synthetic (no BASELINE config)"))

    at = (2, 2, 128, 1024) if small else (32, 32, 512, 1024)      # batch, heads, seq, embed

    def make_attn(u):
        return tuple(u(at, 1552 + i).half() for i in range(3))
    P.append(Problem(97, "x".join(map(str, at)), make_attn, ck.p97.fused_attention_cuda,
                     lambda q, k, v: F.scaled_dot_product_attention(q, k, v),
                     4.0 * at[0] * at[1] * at[2] * at[2] * at[3], k_norm=1,
                     note="fp16; shape within the reference's limits (seq <= 512, embed 1024)"))
    return P


def _time_reps(fn, args, reps: int) -> float:
    """Mean ms per call of ``reps`` back-to-back calls between HIP events."""
    import torch
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn(*args)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _time_pair(ref, ours, args, warmup: int, reps: int, rounds: int):
    """(torch ms, ours ms): warm-up calls of both, then ``rounds`` rounds that
    time ``reps`` calls of each, alternating which goes first; the median
    over the rounds of each one's mean per call."""
    import statistics
    import torch
    for fn in (ref, ours):
        for _ in range(warmup):
            fn(*args)
    torch.cuda.synchronize()
    t_ref, t_ours = [], []
    for r in range(max(1, rounds)):
        if r % 2 == 0:
            t_ref.append(_time_reps(ref, args, reps))
            t_ours.append(_time_reps(ours, args, reps))
        else:
            t_ours.append(_time_reps(ours, args, reps))
            t_ref.append(_time_reps(ref, args, reps))
    return statistics.median(t_ref), statistics.median(t_ours)


def _norm_diff(got, ref, inputs, k: int) -> float:
    """max |got - ref| / (sqrt(K) * max|A| * max|B|) over the tensors given."""
    import torch
    tens = [t for t in inputs if isinstance(t, torch.Tensor) and t.numel()]
    scale = 1.0
    for t in tens[:2]:
        scale *= max(float(t.abs().max()), 1e-30)
    d = float((got.float() - ref.float()).abs().max()) if got.numel() else 0.0
    return d / (math.sqrt(max(k, 1)) * scale)


def run(pids: Optional[Sequence[int]] = None, preset: str = "baseline", warmup: int = 3,
        reps: int = 10, cpu: bool = False, log=print, rounds: int = 5) -> List[Dict[str, object]]:
    """Measure every problem (or ``pids``); returns one row dict per problem."""
    import ctypes
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("evaluate.py needs a HIP device")
    pkg = sys.modules[__package__] if __package__ else None
    ck = pkg if pkg is not None else _load()
    L = ck.abi.lib()
    dev = torch.device("cuda", torch.cuda.current_device())

    def u(shape, seed):
        t = torch.empty(shape, device=dev)
        ck.abi.check(L.mi_fill_uniform_f32(ctypes.c_void_p(t.data_ptr()), t.numel(), seed, 0,
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                     "fill")
        return t

    rows = []
    todo = [p for p in _problems(ck, preset) if not pids or p.pid in pids]
    for p in todo:
        inputs = p.make(u)
        torch.cuda.synchronize()
        t_ref, t_ours = _time_pair(p.torch_ref, p.ours, inputs, warmup, reps, rounds)
        got, ref = p.ours(*inputs), p.torch_ref(*inputs)
        torch.cuda.synchronize()
        diff = _norm_diff(got, ref, inputs, p.k_norm)
        del got, ref
        if p.nbytes:
            thr, unit = p.nbytes / (t_ours * 1e-3) / 1e9, "GB/s"
        else:
            thr, unit = p.flops / (t_ours * 1e-3) / 1e12, "TFLOP/s"
        row = {
            "Problem_ID": p.pid, "Kernels": KERNELS_LABEL,
            "Target_PyTorch_Latency(ms)": t_ref, "Generated_Kernel_Latency(ms)": t_ours,
            "Ratio_to_Target": t_ref / t_ours if t_ours > 0 else float("nan"),
            "Shape": p.shape, "Work": p.note, "Generated_Throughput": thr, "Unit": unit,
            "Max_Norm_Diff_vs_Torch": diff, "CPU_Torch_Latency(ms)": None, "CPU_Threads": None,
        }
        rows.append(row)
        log(f"[eval] PID {p.pid:3d} {p.shape:>24s}: torch {t_ref:9.4f} ms  ours {t_ours:9.4f} ms  "
            f"ratio {row['Ratio_to_Target']:6.2f}  {thr:8.1f} {unit}  diff {diff:.2e}")
        del inputs
        torch.cuda.empty_cache()
    if cpu:
        # host legs after every GPU timing: the host BLAS leaves its threads
        # spinning on every core for a while, which delays GPU launches
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        for p, row in zip(todo, rows):
            inputs = p.make(u)
            host = [t.cpu() if isinstance(t, torch.Tensor) else t for t in inputs]
            del inputs
            torch.cuda.empty_cache()
            p.torch_ref(*host)                      # one warm-up call, then the best of 3
            best = float("inf")
            for _ in range(3):
                t0 = time.perf_counter()
                p.torch_ref(*host)
                best = min(best, time.perf_counter() - t0)
            row["CPU_Torch_Latency(ms)"], row["CPU_Threads"] = best * 1e3, threads
            log(f"[eval] PID {p.pid:3d} host torch {best * 1e3:9.2f} ms on {threads} threads")
            del host
    return rows


def write_csv(rows: Sequence[Dict[str, object]], path: str, extended: bool = False) -> None:
    """The reference's table schema (5 columns), or the extended one."""
    cols = EXT_HEADER if extended else HEADER
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        for r in rows:
            out = []
            for c in cols:
                v = r.get(c)
                if isinstance(v, float):
                    v = f"{v:.6g}" if c in ("Max_Norm_Diff_vs_Torch",) else repr(round(v, 6))
                out.append("" if v is None else v)
            w.writerow(out)


def _load():
    here = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, os.path.dirname(here))
    import __graft_entry__
    return __graft_entry__.load_package()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", default="latency_summary_mi355x.csv",
                    help="reference-schema CSV; the extended table goes next to it (*_ext.csv)")
    ap.add_argument("--pids", default="", help="comma-separated problem ids (default: all)")
    ap.add_argument("--preset", choices=["baseline", "small"], default="baseline")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--rounds", type=int, default=5,
                    help="alternating timing rounds per operator (median reported)")
    ap.add_argument("--cpu", action="store_true", help="also time the torch operator on the host")
    a = ap.parse_args(argv)
    pids = [int(x) for x in a.pids.split(",") if x.strip()]
    rows = run(pids, a.preset, a.warmup, a.reps, a.cpu,
               log=lambda m: print(m, file=sys.stderr, flush=True), rounds=a.rounds)
    write_csv(rows, a.out)
    root, ext = os.path.splitext(a.out)
    write_csv(rows, root + "_ext" + (ext or ".csv"), extended=True)
    print(a.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
