"""Benchmark of the GEMM-family hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--mode full|gemm|gemv|copy]

One step = the BASELINE configs[1] workload: an fp32 8192^3 GEMM in each of the
four operand layouts (A.B, A^T.B, A.B^T, A^T.B^T), run through the drop-in
operators of reference PIDs 1, 16, 17 and 18 on synthetic uniform[-1, 1)
inputs already resident in HBM.  ``value`` is the step's aggregate fp32
TFLOP/s.  The line also carries:
  * ``roofline``: the NN contraction kernel's algorithmic flops per launch
    over its average duration, measured with HIP events on the launch stream
    inside the timed region, against the 157.3 TFLOP/s fp32 MFMA peak;
    ``traffic`` is read from the rocprofv3 PMC summary in profiles/ when present;
  * ``gemv``: the BASELINE GEMV (A 32768 x 65536) in GB/s against 8 TB/s HBM;
  * ``cpu_baseline``: host fp32 torch.matmul (the CPU operator the reference's
    kernels replace) on the same 8192^3 problem, timed on this host's cores.
Only one GPU is supported: --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
METRIC = "fp32 TFLOP/s (% MFMA peak) @8192³ GEMM; GB/s (% HBM peak) on GEMV"
PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
N = 8192
GEMV_M, GEMV_K = 32768, 65536
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemm_f32_nn_8192_traffic.txt")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--mode", choices=["full", "gemm", "gemv", "configs", "copy"], default="full",
                   help="profiling variants: only the GEMM, only the GEMV, only the per-config "
                        "table, or a plain 1 GiB device copy (PMC calibration)")
    p.add_argument("--no-configs", action="store_true", help="skip the per-config table")
    return p.parse_args()


def read_traffic():
    """HBM bytes per NN 8192^3 launch from the committed PMC summary, or None."""
    try:
        txt = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
    return float(m.group(1)) if m else None


# tile configuration of each scheduler plan id (mi_plan.plan_id), as named in
# the kernel symbols rocprofv3 reports
PLAN_KERNELS = {
    1: "gemm_f32_kernel<Tile<64,64,32,32,16,8,2>>",
    2: "gemm_f32_direct_kernel<Tile<128,128,64,64,16,3,2>> (gemm_f32_kernel where direct staging does not apply)",
    3: "gemm_f32_direct_kernel<Tile<256,256,128,64,32,2,2>> (gemm_f32_kernel where direct staging does not apply)",
    4: "gemm_f32_kernel<Tile<128,128,64,64,32,3,1>>",
    5: "gemm_f32_kernel<Tile<128,128,64,64,64,2,1>>",
    6: "gemm_f32_panel_kernel<PanelTile<256,128,32>>",
    7: "gemm_f32_panel_kernel<PanelTile<256,128,64>>",
    8: "gemm_f32_panel_kernel<PanelTile<128,128,64,64,32>>",
}


def nn_kernel_name(ck) -> str:
    """Kernel the scheduler picks for the NN 8192^3 launch, spelled as rocprof
    prints it (N/N launches of the 256 tile with 16-byte operands, K % 32 == 0
    and K >= 256 per split take the direct-staging kernel; template arguments
    <tile, A transposed, B transposed, row bias, structure, bytes per load>)."""
    rc, plan = ck.abi.plan(N, N, N)
    ck.abi.check(rc, "mi_gemm_plan")
    if plan.plan_id == 3 and N % 32 == 0 and plan.k_chunk >= 256:
        return ("mi::gemm_f32_direct_kernel<mi::Tile<256, 256, 128, 64, 32, 2, 2>, false, false, false, 0, 16>"
                f" (split_k {plan.split_k})")
    return f"mi::{PLAN_KERNELS.get(plan.plan_id, plan.plan_id)}, NN, vec4, dense (split_k {plan.split_k})"


def _time(fn, stream, reps, warm):
    import torch
    for _ in range(warm):
        fn(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        fn(i + 1)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def run_configs(ck, fill, dev, stream):
    """Every other BASELINE config at full size, through its operator: ms per
    call and throughput in the config's unit (algorithmic flops or bytes)."""
    import torch
    res = {}

    def rec(name, ms, flops=None, nbytes=None, peak=PEAK_TFLOPS):
        r = {"ms": round(ms, 4)}
        if flops is not None:
            r["tflops"] = round(flops / (ms * 1e-3) / 1e12, 2)
            r["frac_mfma"] = round(r["tflops"] / peak, 4)
        if nbytes is not None:
            r["gbps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            r["frac_hbm"] = round(r["gbps"] / PEAK_HBM_GBS, 4)
        res[name] = r
        log(f"config {name}: {r}")

    def u(shape, seed):
        return fill(torch.empty(shape, device=dev), seed)

    A, B = u((1024, 1024), 0), u((1024, 1024), 1)
    rec("cfg0_nn_1024", _time(lambda i: ck.p01.matmul_cuda(A, B), stream, 20, 3), 2 * 1024 ** 3)
    A, B = u((128, 512, 1024), 32), u((128, 1024, 768), 33)
    rec("batched_128x512x1024x768", _time(lambda i: ck.p03.batched_matmul_cuda(A, B), stream, 10, 2),
        2 * 128 * 512 * 1024 * 768)
    A, B = u((16, 1024, 2048), 34), u((2048, 768), 35)
    rec("tensor3d_16x1024x2048x768", _time(lambda i: ck.p10.batched_matmul_cuda(A, B), stream, 10, 2),
        2 * 16 * 1024 * 2048 * 768)
    A, B = u((8, 64, 128, 256), 36), u((256, 512), 37)
    rec("tensor4d_8x64x128x256x512", _time(lambda i: ck.p11.tensor_matmul_cuda(A, B), stream, 10, 2),
        2 * 65536 * 256 * 512)
    A, B = u((16384, 32), 51), u((32, 16384), 52)
    rec("small_k_16384x16384x32", _time(lambda i: ck.p07.gemm_cuda(A, B), stream, 10, 2),
        2 * 16384 * 16384 * 32, 4 * (2 * 16384 * 32 + 16384 * 16384))
    # diag: two input/output sets (1 GiB in all) alternate so the 256 MB MALL
    # cannot serve a repeat from cache
    a2 = [u((8192,), 53), u((8192,), 55)]
    B2 = [u((8192, 8192), 54), u((8192, 8192), 56)]
    rec("diag_8192", _time(lambda i: ck.p12.diag_mult_cuda(a2[i % 2], B2[i % 2]), stream, 20, 4),
        None, 4 * (8192 + 2 * 8192 * 8192))
    del a2, B2
    # PID 5 matrix-scalar (no BASELINE config names a shape): a 256 MiB matrix,
    # two alternating inputs for the same reason as diag
    A2 = [u((16384, 4096), 57), u((16384, 4096), 58)]
    rec("scalar_16384x4096", _time(lambda i: ck.p05.matrix_scalar_mult_cuda(A2[i % 2], 3.14), stream,
                                   20, 4), None, 4 * 2 * 16384 * 4096)
    del A2
    # PID 87 pointwise conv (no BASELINE config): 16 images of 64 x 256 x 256
    # to 128 channels, with bias; a batched contraction over the weight
    X, W, Bi = u((16, 64, 256, 256), 59), u((128, 64, 1, 1), 60), u((128,), 61)
    rec("pointwise_conv_16x64x128x256x256",
        _time(lambda i: ck.p87.pointwise_conv_cuda(X, W, Bi), stream, 10, 2),
        2 * 16 * 128 * 64 * 65536, 4 * (16 * 64 * 65536 + 128 * 64 + 128 + 16 * 128 * 65536))
    del X, W, Bi
    # PID 97 attention (no BASELINE config): fp16 Q, K, V of 32 x 32 heads x
    # 512 x 1024 (the reference's limits); algorithmic 4 B H S^2 E flops against
    # the fp16 dense MFMA peak
    at = (32, 32, 512, 1024)
    Q, Kt, V = (u(at, 62 + i).half() for i in range(3))
    rec("attention_fp16_32x32x512x1024", _time(lambda i: ck.p97.fused_attention_cuda(Q, Kt, V), stream, 5, 2),
        4.0 * at[0] * at[1] * at[2] ** 2 * at[3], None, PEAK_FP16_TFLOPS)
    del Q, Kt, V
    torch.cuda.empty_cache()
    A, B = u((256, 1 << 20), 64), u((1 << 20, 256), 65)
    rec("large_k_256x256x1048576", _time(lambda i: ck.p06.matmul_cuda(A, B), stream, 10, 2),
        2 * 256 * 256 * (1 << 20))
    del A, B
    A, B = u((65536, 64), 66), u((64, 65536), 67)
    rec("tall_skinny_65536x64", _time(lambda i: ck.p09.tall_skinny_matmul_cuda(A, B), stream, 5, 1),
        2 * 65536 * 65536 * 64, 4 * (2 * 65536 * 64 + 65536 * 65536))
    torch.cuda.empty_cache()
    n = 8192
    tri_flops = n * (n + 1) * (n + 2) / 3
    A, B = torch.tril(u((n, n), 68)), torch.tril(u((n, n), 69))
    rec("lower_tri_8192", _time(lambda i: ck.p15.lower_tri_mul_cuda(A, B), stream, 10, 2), tri_flops)
    A, B = torch.triu(u((n, n), 68)), torch.triu(u((n, n), 69))
    rec("upper_tri_8192", _time(lambda i: ck.p14.upper_tri_matmul_cuda(A, B), stream, 10, 2), tri_flops)
    R1, R2 = u((n, n), 70), u((n, n), 71)
    A, B = (R1 + R1.t()) / 2, (R2 + R2.t()) / 2
    del R1, R2
    rec("symmetric_8192", _time(lambda i: ck.p13.symmetric_matmul_cuda(A, B), stream, 10, 2), 2 * n ** 3)
    del A, B
    torch.cuda.empty_cache()
    return res


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the GEMM-family path has no multi-GPU leg here.", file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, REPO)
    import __graft_entry__

    ck = __graft_entry__.load_package()
    L = ck.abi.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    def fill(t, seed):
        import ctypes
        ck.abi.check(L.mi_fill_uniform_f32(ctypes.c_void_p(t.data_ptr()), t.numel(), seed, 0,
                                           ctypes.c_void_p(stream.cuda_stream)), "fill")
        return t

    if args.mode == "copy":
        src = torch.empty(1 << 28, device=dev)
        dst = torch.empty_like(src)
        fill(src, 5)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy: 1 GiB read + 1 GiB write x3")
        return 0

    out = {}
    if args.mode in ("full", "gemm"):
        # BASELINE seeds: 16 * cfg_index + tensor_index, configs[1] -> 16 (A), 17 (B)
        A = fill(torch.empty((N, N), device=dev), 16)
        B = fill(torch.empty((N, N), device=dev), 17)
        layouts = [("NN", ck.p01.matmul_cuda), ("TN", ck.p16.matmul_transposed_cuda),
                   ("NT", ck.p17.matmul_cuda), ("TT", ck.p18.matmul_transposed_cuda)]
        for _ in range(args.warmup):
            for _, fn in layouts:
                fn(A, B)
        torch.cuda.synchronize()
        n_ev = args.steps * len(layouts) + 1
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        evs[0].record(stream)
        i = 1
        for _ in range(args.steps):
            for _, fn in layouts:
                fn(A, B)
                evs[i].record(stream)
                i += 1
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per = [[] for _ in layouts]
        for s in range(args.steps):
            for j in range(len(layouts)):
                k = 1 + s * len(layouts) + j
                per[j].append(evs[k - 1].elapsed_time(evs[k]))
        step_ms = evs[0].elapsed_time(evs[-1]) / args.steps
        flops = 2.0 * N ** 3
        out["gemm"] = {
            "step_ms": step_ms,
            "wall_ms_per_step": wall * 1e3 / args.steps,
            "tflops": len(layouts) * flops / (step_ms * 1e-3) / 1e12,
            "per_layout_ms": {name: sum(v) / len(v) for (name, _), v in zip(layouts, per)},
        }
        out["gemm"]["per_layout_tflops"] = {
            k: flops / (v * 1e-3) / 1e12 for k, v in out["gemm"]["per_layout_ms"].items()}
        nn_ms = out["gemm"]["per_layout_ms"]["NN"]
        out["roofline"] = {
            "bound": "mfma",
            "kernel": nn_kernel_name(ck),
            "achieved": flops / (nn_ms * 1e-3) / 1e12,
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": flops / (nn_ms * 1e-3) / 1e12 / PEAK_TFLOPS,
            "traffic": read_traffic(),
            "algorithmic_flops_per_launch": flops,
            "avg_launch_ms": nn_ms,
        }
        log(f"gemm 8192^3: step {step_ms:.3f} ms, {out['gemm']['tflops']:.1f} TFLOP/s "
            f"{out['gemm']['per_layout_tflops']}")
        del A, B
        torch.cuda.empty_cache()

    if args.mode in ("full", "gemv"):
        import ctypes
        A = fill(torch.empty((GEMV_M, GEMV_K), device=dev), 48)   # configs[3] -> 48 (A)
        x = fill(torch.empty((GEMV_K, 1), device=dev), 50)        # x -> 50
        # the first passes over a fresh 8 GiB operand run slower (page and
        # clock warm-up: ~1.7 ms on the first call, ~1.25 ms after ~30)
        for _ in range(max(args.warmup, 30)):
            ck.p04.gemv_cuda(A, x)
        torch.cuda.synchronize()
        reps = max(args.steps, 20)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            ck.p04.gemv_cuda(A, x)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        nbytes = (GEMV_M * GEMV_K + GEMV_K + GEMV_M) * 4
        out["gemv"] = {"shape": [GEMV_M, GEMV_K], "ms": ms, "gbps": nbytes / (ms * 1e-3) / 1e9,
                       "frac": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                       "algorithmic_bytes": nbytes}
        log(f"gemv {GEMV_M}x{GEMV_K}: {ms:.3f} ms, {out['gemv']['gbps']:.0f} GB/s")
        del A, x
        torch.cuda.empty_cache()

    if args.mode in ("full", "configs") and not args.no_configs:
        out["configs"] = run_configs(ck, fill, dev, stream)

    if args.mode != "full":
        return 0

    cpu = None
    if not args.no_cpu:
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        a = torch.rand((N, N)) * 2 - 1
        b = torch.rand((N, N)) * 2 - 1
        torch.matmul(a[:512], b)  # warm the BLAS thread pool
        # one bench step on the host: the same four 8192^3 layouts (A.B, A^T.B,
        # A.B^T, A^T.B^T through transposed views), best of 2 steps
        best = float("inf")
        for _ in range(2):
            t = time.perf_counter()
            for x, y in ((a, b), (a.t(), b), (a, b.t()), (a.t(), b.t())):
                torch.matmul(x, y)
            best = min(best, time.perf_counter() - t)
        cpu = {"value": 4 * 2.0 * N ** 3 / best / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
               "kind": "reference",
               "sample": f"one bench step on the host: fp32 torch.matmul 8192^3 in the four layouts "
                         f"NN/TN/NT/TT (the CPU operator the reference's kernels replace), best of 2 "
                         f"steps after a warm-up, {best * 1e3:.0f} ms per step; torch {torch.__version__}"}
        log(f"cpu baseline: {cpu['value']:.3f} TFLOP/s on {cpu['cores']} threads")

    g = out["gemm"]
    line = {
        "metric": METRIC,
        "value": round(g["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "fp32 GEMM M=N=K=8192 in layouts NN, TN, NT, TT "
                               "(BASELINE configs[1]); one step = one GEMM per layout",
                   "M": N, "N": N, "K": N, "layouts": ["NN", "TN", "NT", "TT"],
                   "inputs": "uniform[-1,1) splitmix64 seeds 16/17, resident in HBM"},
        "frac_of_peak": round(g["tflops"] / PEAK_TFLOPS, 4),
        "per_layout_tflops": {k: round(v, 2) for k, v in g["per_layout_tflops"].items()},
        "roofline": out["roofline"],
        "gemv": out.get("gemv"),
        "configs": out.get("configs"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
