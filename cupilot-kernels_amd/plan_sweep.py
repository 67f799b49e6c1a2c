"""Time candidate plans of mi_gemm_f32 on this GPU, for refitting the planner's
cost model (csrc/scheduler.cpp, kModels).

For every shape it forces each plan_override in turn (tile config | split-K
<< 8 | stream-K bit 0x10), skips overrides that resolve to a plan already
timed, and times the plan with HIP events over back-to-back calls (median of
ROUNDS rounds, after one untimed round).  Output: CSV rows in the format of
tests/data/plan_timings_mi355x.csv.

usage: python cupilot-kernels_amd/plan_sweep.py OUT.csv [--rounds 3] [--shapes FILE]
       [--overrides 0,0x3,...]
FILE: one shape per line, MxNxK[xBATCH][:LAYOUT] (LAYOUT NN, TN, NT or TT).
"""
from __future__ import annotations

import argparse
import ctypes
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import torch  # noqa: E402  (binds the HIP runtime before the library loads)

import abi  # noqa: E402

DEFAULT_OVERRIDES = [0, 0x3, 0x203, 0x403, 0x803, 0x2, 0x202, 0x402, 0x802, 0x1002, 0x9, 0x209, 0x409,
                     0x809, 0x1009, 0x1, 0x201, 0x401, 0x801, 0x13, 0x12, 0x19]
DEFAULT_SHAPES = ["1024x1024x1024", "2048x2048x2048", "2048x4096x2048", "3072x3072x3072",
                  "3072x3072x8192", "4608x4608x4608", "8192x8192x8192", "65536x512x256",
                  "16384x768x2048", "2048x8192x4096", "1280x1280x8192", "512x512x32768"]


def parse_shape(text):
    dims, _, lay = text.strip().partition(":")
    v = [int(x) for x in dims.split("x")]
    return v[0], v[1], v[2], (v[3] if len(v) > 3 else 1), (lay or "NN")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("out")
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--shapes", default=None)
    ap.add_argument("--overrides", default=None)
    args = ap.parse_args(argv)
    shapes = [parse_shape(s) for s in (open(args.shapes) if args.shapes else DEFAULT_SHAPES) if s.strip()]
    overrides = [int(v, 0) for v in args.overrides.split(",")] if args.overrides else DEFAULT_OVERRIDES
    L = abi.lib()
    st = torch.cuda.current_stream()
    sp = ctypes.c_void_p(st.cuda_stream)
    with open(args.out, "w") as out:
        out.write("M,N,K,batch,layout,cfg,split,stream_k,ms\n")
        for M, N, K, batch, lay in shapes:
            oa, ob = int(lay[0] == "T"), int(lay[1] == "T")
            A = torch.empty((batch,) + ((K, M) if oa else (M, K)), device="cuda")
            B = torch.empty((batch,) + ((N, K) if ob else (K, N)), device="cuda")
            C = torch.empty((batch, M, N), device="cuda")
            abi.check(L.mi_fill_uniform_f32(A.data_ptr(), A.numel(), 1, 0, sp))
            abi.check(L.mi_fill_uniform_f32(B.data_ptr(), B.numel(), 2, 0, sp))
            seen = {}
            for ov in overrides:
                a = abi.make_args(M, N, K, batch=batch, op_a=oa, op_b=ob, plan_override=ov,
                                  workspace_bytes=1 << 40)
                a.stride_a, a.stride_b, a.stride_c = M * K, K * N, M * N
                p = abi.Plan()
                if L.mi_gemm_plan(ctypes.byref(a), 256, ctypes.byref(p)) != abi.MI_OK:
                    continue
                key = (p.plan_id, p.split_k, p.stream_k)
                if key in seen:
                    continue
                ws = torch.empty(max(p.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
                a.A, a.B, a.C = A.data_ptr(), B.data_ptr(), C.data_ptr()
                a.workspace, a.workspace_bytes = ws.data_ptr(), p.workspace_bytes
                reps = max(3, min(40, int(2e10 / (2.0 * batch * M * N * K / 1e3))))
                for _ in range(reps):
                    abi.check(L.mi_gemm_f32(ctypes.byref(a), sp), "mi_gemm_f32")
                torch.cuda.synchronize()
                times = []
                for _ in range(args.rounds):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(st)
                    for _ in range(reps):
                        L.mi_gemm_f32(ctypes.byref(a), sp)
                    e1.record(st)
                    torch.cuda.synchronize()
                    times.append(e0.elapsed_time(e1) / reps)
                seen[key] = statistics.median(times)
                out.write(f"{M},{N},{K},{batch},{lay},{key[0]},{key[1]},{key[2]},{seen[key]:.6f}\n")
                out.flush()
                del ws
            flops = 2.0 * batch * M * N * K
            print(f"{M}x{N}x{K}x{batch}:{lay} " + " ".join(
                f"{c}/{s}{'s' if k else ''}:{flops / t / 1e9:.0f}" for (c, s, k), t in seen.items()), flush=True)
            del A, B, C
            torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
