"""Benchmark of the GEMM-family hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-configs]
    python bench.py --mode NAME [--steps K] [--warmup W]     one config alone (profiling)
    python bench.py --mode list                              the config names
    python bench.py --mode gemm:MxNxK[:TN|NT|TT][@BITS][,...] [--override BITS]
    python bench.py --mode torch:MxNxK[:TN|NT|TT][,...]     (torch-ROCm's own GEMM, for profiling)
                                                    dense products through the C ABI, with a
                                                    plan override (stream-K / tile / split);
                                                    --mode runs keep exactly --warmup calls
                                                    per entry: with few (5), the first entry
                                                    after a change of shape measured up to
                                                    ~2 % slow, so compare plans with >= 30
    python bench.py --summarize DIR [DIR ...] [--calib DIR]  rocprofv3 CSV output -> text summary

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
  * ``configs``: every other BASELINE config at full size through its
    operator, each with the host CPU time of the torch operator it replaces
    (``cpu``), on the same inputs;
  * ``cpu_baseline``: host fp32 torch.matmul (the CPU operator the reference's
    kernels replace) on one bench step, timed on this host's cores;
  * ``host``: nproc, CPU model, torch and BLAS versions.
Only one GPU is supported: --gpus N with N > 1 exits with a message.

``--mode NAME`` runs one config (W untimed calls, then K timed calls) and prints
one JSON line; ``rocprofv3 ... -- python bench.py --mode NAME`` profiles that
config alone.  ``--summarize`` turns the CSV files rocprofv3 wrote
(``--output-format csv``) into the text summaries kept in profiles/: kernel
durations averaged over the last K dispatches of each kernel (the timed ones),
and per-dispatch counters (MFMA busy, fp32 MFMA flops, engine clock, L2 hit
rate, HBM bytes scaled by a plain-copy calibration).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import platform
import re
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
METRIC = "fp32 TFLOP/s (% MFMA peak) @8192³ GEMM; GB/s (% HBM peak) on GEMV"
PEAK_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
NUM_XCD, NUM_SIMD = 8, 1024  # MI355X: 8 XCDs, 256 CUs x 4 SIMDs
N = 8192
GEMV_M, GEMV_K = 32768, 65536
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemm_f32_nn_8192.txt")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--no-cpu", action="store_true", help="skip every CPU baseline")
    p.add_argument("--mode", default="full",
                   help="full (default), gemm (the headline step only), configs (the per-config "
                        "table only), copy (a plain 1 GiB device copy: PMC calibration), list, or "
                        "one config name")
    p.add_argument("--no-configs", action="store_true", help="skip the per-config table")
    p.add_argument("--override", type=lambda x: int(x, 0), default=0,
                   help="with --mode gemm:MxNxK[:TN|NT|TT]: mi_gemm_args.plan_override (bits 0-3 tile "
                        "config, 4 take stream-K, 5 no stream-K, 8-19 split count, 30 stream-K over "
                        "contiguous ranges instead of phases)")
    p.add_argument("--summarize", nargs="+", metavar="DIR",
                   help="summarise rocprofv3 CSV output under DIR(s) and exit")
    p.add_argument("--calib", metavar="DIR", default=None,
                   help="with --summarize: rocprofv3 FETCH_SIZE / WRITE_SIZE output of --mode copy")
    return p.parse_args()


def read_traffic():
    """HBM bytes per NN 8192^3 launch from the committed PMC summary, or None."""
    try:
        txt = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
    return float(m.group(1)) if m else None


def host_info():
    import torch
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        m = re.search(r"^Model name:\s*(.+)$", out, re.M)
        model = m.group(1).strip() if m else None
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None:
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    cfg = torch.__config__.show()
    blas = re.search(r"BLAS_INFO=(\w+)", cfg)
    mkl = re.search(r"Intel\(R\) (?:oneAPI )?Math Kernel Library Version ([0-9.]+)", cfg)
    return {"nproc": os.cpu_count(), "cpu_model": model or platform.processor(),
            "torch": torch.__version__, "blas": (blas.group(1) if blas else None),
            "mkl": (mkl.group(1) if mkl else None), "threads": torch.get_num_threads()}


# ---------------------------------------------------------------------------
# configs
# ---------------------------------------------------------------------------
class Cfg:
    """One workload: inputs (device), the operator, its algorithmic work and
    the host torch operator it replaces.  ``sets`` > 1 rotates input sets so
    that a bandwidth-bound call cannot find its operands in the 256 MB MALL."""

    def __init__(self, name, make, op, cpu, flops=None, nbytes=None, peak=PEAK_TFLOPS,
                 reps=10, warmup=2, sets=1, cpu_note="", cpu_scale=1.0, cpu_sample=None,
                 baseline=True):
        self.name, self.make, self.op, self.cpu = name, make, op, cpu
        self.flops, self.nbytes, self.peak = flops, nbytes, peak
        self.reps, self.warmup, self.sets = reps, warmup, sets
        self.cpu_note, self.cpu_scale, self.cpu_sample = cpu_note, cpu_scale, cpu_sample
        self.baseline = baseline


def configs(ck):
    import torch
    import torch.nn.functional as F

    n = N
    tri_flops = n * (n + 1) * (n + 2) / 3
    C = []

    def add(*a, **k):
        C.append(Cfg(*a, **k))

    # BASELINE seeds: 16 * cfg_index + tensor_index (A = 0, B = 1, x/a = 2, R = 3)
    add("cfg0_nn_1024", lambda u: (u((1024, 1024), 0), u((1024, 1024), 1)),
        lambda a, b: ck.p01.matmul_cuda(a, b), lambda a, b: a @ b, flops=2 * 1024 ** 3, reps=50,
        warmup=5, cpu_note="A @ B")
    for lay, fn, cpu in (("nn", ck.p01.matmul_cuda, lambda a, b: a @ b),
                         ("tn", ck.p16.matmul_transposed_cuda, lambda a, b: a.t() @ b),
                         ("nt", ck.p17.matmul_cuda, lambda a, b: a @ b.t()),
                         ("tt", ck.p18.matmul_transposed_cuda, lambda a, b: a.t() @ b.t())):
        add(f"gemm_{lay}_8192", lambda u: (u((n, n), 16), u((n, n), 17)), fn, cpu,
            flops=2 * n ** 3, reps=5, warmup=2,
            cpu_note={"nn": "A @ B", "tn": "A.T @ B (A stored KxM)", "nt": "A @ B.T (B stored NxK)",
                      "tt": "A.T @ B.T"}[lay])
    add("batched_128x512x1024x768", lambda u: (u((128, 512, 1024), 32), u((128, 1024, 768), 33)),
        lambda a, b: ck.p03.batched_matmul_cuda(a, b), lambda a, b: torch.bmm(a, b),
        flops=2 * 128 * 512 * 1024 * 768, cpu_note="torch.bmm(A, B)")
    add("tensor3d_16x1024x2048x768", lambda u: (u((16, 1024, 2048), 34), u((2048, 768), 35)),
        lambda a, b: ck.p10.batched_matmul_cuda(a, b), lambda a, b: torch.matmul(a, b),
        flops=2 * 16 * 1024 * 2048 * 768, cpu_note="torch.matmul(A, B), A 3-D")
    add("tensor4d_8x64x128x256x512", lambda u: (u((8, 64, 128, 256), 36), u((256, 512), 37)),
        lambda a, b: ck.p11.tensor_matmul_cuda(a, b),
        lambda a, b: torch.einsum("bijl,lk->bijk", a, b), flops=2 * 65536 * 256 * 512,
        cpu_note="torch.einsum('bijl,lk->bijk', A, B)")
    add("gemv_32768x65536", lambda u: (u((GEMV_M, GEMV_K), 48), u((GEMV_K, 1), 50)),
        lambda a, x: ck.p04.gemv_cuda(a, x), lambda a, x: a @ x,
        nbytes=4 * (GEMV_M * GEMV_K + GEMV_K + GEMV_M), reps=20, warmup=30, cpu_note="A @ x")
    add("small_k_16384x16384x32", lambda u: (u((16384, 32), 51), u((32, 16384), 52)),
        lambda a, b: ck.p07.gemm_cuda(a, b), lambda a, b: a @ b, flops=2 * 16384 * 16384 * 32,
        nbytes=4 * (2 * 16384 * 32 + 16384 * 16384), cpu_note="A @ B")
    add("diag_8192", lambda u: (u((n,), 53), u((n, n), 54)),
        lambda a, b: ck.p12.diag_mult_cuda(a, b), lambda a, b: torch.diag(a) @ b,
        nbytes=4 * (n + 2 * n * n), reps=20, warmup=4, sets=2,
        cpu_note="torch.diag(a) @ B (the reference's torch formulation, a full GEMM)")
    add("large_k_256x256x1048576", lambda u: (u((256, 1 << 20), 64), u((1 << 20, 256), 65)),
        lambda a, b: ck.p06.matmul_cuda(a, b), lambda a, b: a @ b, flops=2 * 256 * 256 * (1 << 20),
        cpu_note="A @ B")
    add("tall_skinny_65536x64", lambda u: (u((65536, 64), 66), u((64, 65536), 67)),
        lambda a, b: ck.p09.tall_skinny_matmul_cuda(a, b), lambda a, b: a[:4096] @ b,
        flops=2 * 65536 * 65536 * 64, nbytes=4 * (2 * 65536 * 64 + 65536 * 65536), reps=5, warmup=1,
        cpu_note="A @ B", cpu_scale=16.0,
        cpu_sample="rows 0-4095 of A (1/16 of the output), time x 16")
    add("lower_tri_8192", lambda u: (torch.tril(u((n, n), 68)), torch.tril(u((n, n), 69))),
        lambda a, b: ck.p15.lower_tri_mul_cuda(a, b), lambda a, b: torch.tril(a @ b),
        flops=tri_flops, cpu_note="torch.tril(A @ B)")
    add("upper_tri_8192", lambda u: (torch.triu(u((n, n), 68)), torch.triu(u((n, n), 69))),
        lambda a, b: ck.p14.upper_tri_matmul_cuda(a, b), lambda a, b: torch.triu(a @ b),
        flops=tri_flops, cpu_note="torch.triu(A @ B)")

    def sym(u):
        r1, r2 = u((n, n), 70), u((n, n), 71)
        return (r1 + r1.t()) / 2, (r2 + r2.t()) / 2
    add("symmetric_8192", sym, lambda a, b: ck.p13.symmetric_matmul_cuda(a, b), lambda a, b: a @ b,
        flops=2 * n ** 3, reps=5, cpu_note="A @ B")
    # not BASELINE configs: the reference's literal PID 2 extents (M = 2048,
    # K = 8192, N = 4096: kernels/2_...:16-18), shapes that show the stream-K
    # schedule, and the next rows (PIDs 5, 87, 97)
    add("pid2_2048x8192x4096", lambda u: (u((2048, 8192), 80), u((8192, 4096), 81)),
        lambda a, b: ck.p02.matmul_cuda(a, b), lambda a, b: a @ b, flops=2 * 2048 * 8192 * 4096,
        cpu_note="A @ B", baseline=False)
    for (m_, n_, k_) in ((3072, 3072, 8192), (4608, 4608, 4608)):
        add(f"stream_k_{m_}x{n_}x{k_}", lambda u, m_=m_, n_=n_, k_=k_: (u((m_, k_), 82), u((k_, n_), 83)),
            lambda a, b: ck.p02.matmul_cuda(a, b), lambda a, b: a @ b, flops=2 * m_ * n_ * k_,
            cpu_note="A @ B", baseline=False)
    # PID 8's irregular extents (M = 8205, K = 2949, N = 5921, the synthetic
    # shape the evaluation runner uses): rows not 16-byte aligned, so the
    # planner packs the operands before the 16-byte kernels run
    add("irregular_8205x2949x5921", lambda u: (u((8205, 2949), 84), u((2949, 5921), 85)),
        lambda a, b: ck.p08.matmul_cuda(a, b), lambda a, b: a @ b, flops=2 * 8205 * 2949 * 5921,
        cpu_note="A @ B", baseline=False)
    add("scalar_16384x4096", lambda u: (u((16384, 4096), 57),),
        lambda a: ck.p05.matrix_scalar_mult_cuda(a, 3.14), lambda a: a * 3.14,
        nbytes=4 * 2 * 16384 * 4096, reps=20, warmup=4, sets=2, cpu_note="A * s", baseline=False)
    add("pointwise_conv_16x64x128x256x256",
        lambda u: (u((16, 64, 256, 256), 59), u((128, 64, 1, 1), 60), u((128,), 61)),
        lambda x, w, b: ck.p87.pointwise_conv_cuda(x, w, b), lambda x, w, b: F.conv2d(x, w, b),
        flops=2 * 16 * 128 * 64 * 65536,
        nbytes=4 * (16 * 64 * 65536 + 128 * 64 + 128 + 16 * 128 * 65536),
        cpu_note="F.conv2d(x, w, b)", baseline=False)
    at = (32, 32, 512, 1024)

    def attn(u):
        return tuple(u(at, 62 + i).half() for i in range(3))
    add("attention_fp16_32x32x512x1024", attn, lambda q, k, v: ck.p97.fused_attention_cuda(q, k, v),
        lambda q, k, v: F.scaled_dot_product_attention(q[:1].float(), k[:1].float(), v[:1].float()),
        flops=4.0 * at[0] * at[1] * at[2] ** 2 * at[3], peak=PEAK_FP16_TFLOPS, reps=5,
        cpu_note="F.scaled_dot_product_attention in fp32", cpu_scale=32.0,
        cpu_sample="batch 0 of 32 (32 heads), time x 32", baseline=False)
    return C


def adhoc_gemm(ck, mode, override):
    """--mode gemm:MxNxK[:TN|NT|TT]: one dense product through the C ABI
    (mi_gemm_f32) with a plan override and a workspace from the plan."""
    import ctypes

    import torch
    parts = mode.split(":")
    M, N_, K = (int(x) for x in parts[1].split("x"))
    lay = parts[2] if len(parts) > 2 else "NN"
    op_a, op_b = int(lay[0] == "T"), int(lay[1] == "T")
    L = ck.abi.lib()
    state = {}

    def make(u):
        a = u((K, M) if op_a else (M, K), 1)
        b = u((N_, K) if op_b else (K, N_), 2)
        c = torch.empty((M, N_), device=a.device)
        args = ck.abi.make_args(M, N_, K, op_a=op_a, op_b=op_b, plan_override=override,
                                workspace_bytes=1 << 40)
        need = L.mi_gemm_workspace_bytes(ctypes.byref(args))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=a.device)
        args.A, args.B, args.C = a.data_ptr(), b.data_ptr(), c.data_ptr()
        args.workspace, args.workspace_bytes = ws.data_ptr(), need
        state["keep"] = (a, b, c, ws)
        return (args,)

    def op(args):
        ck.abi.check(L.mi_gemm_f32(ctypes.byref(args),
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "mi_gemm_f32")
    c = Cfg(mode, make, op, None, flops=2.0 * M * N_ * K, baseline=False)
    c.M, c.N, c.K, c.op_a, c.op_b = M, N_, K, op_a, op_b
    return c


def adhoc_torch_gemm(mode):
    """--mode torch:MxNxK[:TN|NT|TT]: the same product through torch-ROCm's
    own GEMM (A @ B on the GPU, transposed views for the T layouts), for
    profiling the library kernel this path is measured against."""
    import torch
    parts = mode.split(":")
    M, N_, K = (int(x) for x in parts[1].split("x"))
    lay = parts[2] if len(parts) > 2 else "NN"
    op_a, op_b = lay[0] == "T", lay[1] == "T"
    state = {}

    def make(u):
        a = u((K, M) if op_a else (M, K), 1)
        b = u((N_, K) if op_b else (K, N_), 2)
        state["keep"] = (a, b)
        return (a.t() if op_a else a, b.t() if op_b else b)

    def op(a, b):
        state["out"] = a @ b
    return Cfg(mode, make, op, None, flops=2.0 * M * N_ * K, baseline=False)


def make_filler(ck, dev, stream):
    import ctypes

    import torch

    L = ck.abi.lib()

    def u(shape, seed):
        t = torch.empty(shape, device=dev)
        ck.abi.check(L.mi_fill_uniform_f32(ctypes.c_void_p(t.data_ptr()), t.numel(), seed, 0,
                                           ctypes.c_void_p(stream.cuda_stream)), "fill")
        return t
    return u


def time_gpu(c, inputs, stream, reps, warmup, warm_ms=50.0):
    """Mean ms per call of c.op over reps calls (HIP events on the launch
    stream) after at least `warmup` untimed calls and at least warm_ms of
    untimed work (the engine clock ramps up from idle over ~40 ms); input
    sets rotate per call."""
    import torch
    t = time.perf_counter()
    c.op(*inputs[0])
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t, 1e-6) * 1e3
    n = max(warmup - 1, int(warm_ms / one) + 1) if warm_ms > 0 else warmup - 1
    for i in range(n):
        c.op(*inputs[(i + 1) % len(inputs)])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        c.op(*inputs[i % len(inputs)])
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_cpu(fn, args, reps=3):
    """Best of reps host calls after one warm-up call (ms)."""
    fn(*args)
    best = float("inf")
    for _ in range(reps):
        t = time.perf_counter()
        fn(*args)
        best = min(best, time.perf_counter() - t)
    return best * 1e3


def rates(c, ms):
    r = {"ms": round(ms, 4)}
    if c.flops is not None:
        r["tflops"] = round(c.flops / (ms * 1e-3) / 1e12, 2)
        r["frac_mfma"] = round(r["tflops"] / c.peak, 4)
    if c.nbytes is not None:
        r["gbps"] = round(c.nbytes / (ms * 1e-3) / 1e9, 1)
        r["frac_hbm"] = round(r["gbps"] / PEAK_HBM_GBS, 4)
    return r


def run_config(c, u, stream, reps=None, warmup=None, exact_warmup=False):
    """GPU time of one config (inputs made on the device, then freed)."""
    import torch
    reps = c.reps if reps is None else reps
    warmup = c.warmup if warmup is None else warmup
    inputs = [c.make(lambda shape, seed, s=s: u(shape, seed + 1000 * s)) for s in range(c.sets)]
    torch.cuda.synchronize()
    # --mode runs (profiling) keep exactly the requested warm-up count, so the
    # timed calls are the last `reps` dispatches of each kernel
    r = rates(c, time_gpu(c, inputs, stream, reps, warmup, 0.0 if exact_warmup else 50.0))
    r["calls"] = {"warmup": warmup if exact_warmup else f">= {warmup} and >= 50 ms", "timed": reps}
    del inputs
    torch.cuda.empty_cache()
    return r


def run_cpu_leg(c, u):
    """Host time of the torch operator a config's kernel replaces, on the same
    inputs (made on the device, copied to the host).  Run after every GPU
    timing: the host BLAS leaves its threads spinning on every core for a
    while, which delays the launching thread of a GPU measurement."""
    import torch
    inputs = c.make(u)
    host = [t.cpu() if isinstance(t, torch.Tensor) else t for t in inputs]
    del inputs
    torch.cuda.empty_cache()
    ms = time_cpu(c.cpu, host) * c.cpu_scale
    cr = {"op": c.cpu_note, "ms": round(ms, 2), "threads": torch.get_num_threads(),
          "best_of": 3, "after_warmup": 1}
    if c.flops is not None:
        cr["tflops"] = round(c.flops / (ms * 1e-3) / 1e12, 4)
    if c.nbytes is not None:
        cr["gbps"] = round(c.nbytes / (ms * 1e-3) / 1e9, 2)
    if c.cpu_sample:
        cr["sample"] = c.cpu_sample
    return cr


# ---------------------------------------------------------------------------
# the headline step
# ---------------------------------------------------------------------------
def nn_kernel_name(ck) -> str:
    """Kernel the scheduler picks for the NN 8192^3 launch, spelled as rocprof
    prints it."""
    rc, plan = ck.abi.plan(N, N, N)
    ck.abi.check(rc, "mi_gemm_plan")
    if plan.plan_id == 3 and N % 32 == 0 and plan.k_chunk >= 256 and not plan.stream_k:
        return ("mi::gemm_f32_direct_kernel<mi::Tile<256, 256, 128, 64, 32, 2, 2>, false, false, false, 0, 16,"
                f" false> (split_k {plan.split_k})")
    return f"plan {plan.plan_id} split_k {plan.split_k} stream_k {plan.stream_k}"


def run_headline(ck, u, stream, steps, warmup):
    import torch
    A, B = u((N, N), 16), u((N, N), 17)   # configs[1] -> seeds 16 (A), 17 (B)
    layouts = [("NN", ck.p01.matmul_cuda), ("TN", ck.p16.matmul_transposed_cuda),
               ("NT", ck.p17.matmul_cuda), ("TT", ck.p18.matmul_transposed_cuda)]
    for _ in range(warmup):
        for _, fn in layouts:
            fn(A, B)
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps * len(layouts) + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record(stream)
    i = 1
    for _ in range(steps):
        for _, fn in layouts:
            fn(A, B)
            evs[i].record(stream)
            i += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [[] for _ in layouts]
    for s in range(steps):
        for j in range(len(layouts)):
            k = 1 + s * len(layouts) + j
            per[j].append(evs[k - 1].elapsed_time(evs[k]))
    step_ms = evs[0].elapsed_time(evs[-1]) / steps
    flops = 2.0 * N ** 3
    g = {"step_ms": step_ms, "wall_ms_per_step": wall * 1e3 / steps,
         "tflops": len(layouts) * flops / (step_ms * 1e-3) / 1e12,
         "per_layout_ms": {name: sum(v) / len(v) for (name, _), v in zip(layouts, per)}}
    g["per_layout_tflops"] = {k: flops / (v * 1e-3) / 1e12 for k, v in g["per_layout_ms"].items()}
    nn_ms = g["per_layout_ms"]["NN"]
    roof = {"bound": "mfma", "kernel": nn_kernel_name(ck),
            "achieved": flops / (nn_ms * 1e-3) / 1e12, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": flops / (nn_ms * 1e-3) / 1e12 / PEAK_TFLOPS, "traffic": read_traffic(),
            "algorithmic_flops_per_launch": flops, "avg_launch_ms": nn_ms,
            "launches_averaged": steps}
    log(f"gemm 8192^3: step {step_ms:.3f} ms, {g['tflops']:.1f} TFLOP/s {g['per_layout_tflops']}")
    del A, B
    torch.cuda.empty_cache()
    return g, roof


def cpu_headline(u):
    """One bench step on the host: the four 8192^3 layouts (transposed views of
    the same seed-16 / seed-17 inputs the GPU step uses), each the best of 3
    calls after one warm-up call."""
    import torch
    a, b = u((N, N), 16).cpu(), u((N, N), 17).cpu()
    per = {}
    for name, (x, y) in (("NN", (a, b)), ("TN", (a.t(), b)), ("NT", (a, b.t())),
                         ("TT", (a.t(), b.t()))):
        per[name] = round(time_cpu(torch.matmul, (x, y)), 1)
    ms = sum(per.values())
    return {"value": 4 * 2.0 * N ** 3 / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "reference",
            "sample": f"one bench step on the host: fp32 torch.matmul 8192^3 in the four layouts "
                      f"NN/TN/NT/TT (the CPU operator the reference's kernels replace), each the "
                      f"best of 3 calls after one warm-up call, {ms:.0f} ms per step",
            "per_layout_ms": per}


# ---------------------------------------------------------------------------
# rocprofv3 CSV summaries
# ---------------------------------------------------------------------------
def _short(name: str) -> str:
    name = re.sub(r"^void ", "", name).replace("mi::", "")
    return re.sub(r"\(.*\)$", "", name)


def _csv_rows(dirs, suffix):
    rows = []
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)):
            rows.extend(csv.DictReader(open(f)))
    return rows


SETUP_KERNELS = ("fill_uniform", "copyBuffer", "at::native")   # inputs, not the operator


def pmc_passes():
    """The counter sets of the per-config profiles, one rocprofv3 run each
    (within the per-block limits: 8 SQ, 4 TCC -- FETCH_SIZE takes 3, WRITE_SIZE 2)."""
    return [["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_MOPS_F16",
             "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "GRBM_GUI_ACTIVE"],
            ["TCC_HIT_sum", "TCC_MISS_sum", "WRITE_SIZE"], ["FETCH_SIZE"]]


def summary_header(cfg, timed, warmup, root):
    """The commands (from the repo root) whose output a summary condenses."""
    d = f"{root}/{cfg.name}"
    run = f"-- python3 bench.py --mode {cfg.name} --steps {timed} --warmup {warmup}"
    lines = [f"rocprofv3 summary -- bench config {cfg.name} on one MI355X (gfx950, 256 CUs, 8 XCDs)",
             "",
             "commands (from the repo root, TMPDIR=/tmp; each rocprofv3 pass is a run of its own):",
             f"  rocprofv3 --kernel-trace --stats --output-format csv -d {d}/trace -o kt {run}"]
    for i, p in enumerate(pmc_passes(), 1):
        lines.append(f"  rocprofv3 --pmc {' '.join(p)} --output-format csv -d {d}/pmc{i} -o p {run}")
    lines += ["  calibration (a plain 1 GiB device copy):",
              f"  rocprofv3 --pmc FETCH_SIZE --output-format csv -d {root}/copy/f -o c -- python3 bench.py --mode copy",
              f"  rocprofv3 --pmc WRITE_SIZE --output-format csv -d {root}/copy/w -o c -- python3 bench.py --mode copy",
              f"  python3 bench.py --summarize {d}/trace {d}/pmc1 {d}/pmc2 {d}/pmc3 --calib {root}/copy "
              f"--mode {cfg.name} --steps {timed} --warmup {warmup}", ""]
    return lines


def _per_call(n_dispatch, timed, warmup):
    """Dispatches of a kernel per operator call in a --mode run of
    warmup + timed calls (1 when the count does not divide evenly)."""
    calls = timed + (warmup or 0)
    if warmup is not None and n_dispatch >= calls and n_dispatch % calls == 0:
        return n_dispatch // calls
    return 1


def summarize(dirs, calib, timed, cfg=None, warmup=None):
    """Text summary of rocprofv3 --output-format csv runs: per kernel, the
    mean over the dispatches of the last `timed` calls of a --mode run of
    warmup + timed calls; with cfg, the operator's time per call (its
    kernels' timed means times their dispatches per call, added) against its
    algorithmic work and roofline."""
    out = []
    means = {}   # kernel -> timed mean (ns), for ordering and picking the main kernel
    trace = _csv_rows(dirs, "_kernel_trace.csv")
    if trace:
        by = {}
        for r in trace:
            by.setdefault(r["Kernel_Name"], []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        out.append(f"kernel durations (us): all dispatches, and the mean over the dispatches of the "
                   f"last {timed} calls (the timed calls)")
        out.append(f"  {'disp':>5} {'per call':>8} {'timed mean':>11} {'min':>9} {'max':>9}  kernel")
        op_us = 0.0
        for k, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
            per_call = _per_call(len(v), timed, warmup)
            last = v[-timed * per_call:] if len(v) >= timed * per_call else v
            mean = sum(last) / len(last) / 1e3
            means[k] = mean * per_call
            out.append(f"  {len(v):5d} {per_call:8d} {mean:11.2f} {min(v) / 1e3:9.2f} {max(v) / 1e3:9.2f}  "
                       f"{_short(k)}")
            if len(v) >= timed and not any(x in k for x in SETUP_KERNELS):
                op_us += mean * per_call
        if cfg is not None and op_us > 0:
            out.append(f"operator time per call (timed means x dispatches per call, added over its kernels): "
                       f"{op_us:.2f} us")
            if cfg.flops is not None:
                tf = cfg.flops / (op_us * 1e-6) / 1e12
                out.append(f"  algorithmic {cfg.flops:.6g} flop -> {tf:.2f} TFLOP/s = {tf / cfg.peak:.3f} of "
                           f"the {cfg.peak} TFLOP/s {'fp16' if cfg.peak == PEAK_FP16_TFLOPS else 'fp32'} "
                           f"MFMA peak")
            if cfg.nbytes is not None:
                gb = cfg.nbytes / (op_us * 1e-6) / 1e9
                out.append(f"  algorithmic {cfg.nbytes:.6g} bytes -> {gb:.1f} GB/s = {gb / PEAK_HBM_GBS:.3f} "
                           f"of the 8 TB/s HBM peak")
    pmc = _csv_rows(dirs, "_counter_collection.csv")
    if pmc:
        scale = {"FETCH_SIZE": 1.0, "WRITE_SIZE": 1.0}
        if calib:
            for cname in scale:
                vals = [float(r["Counter_Value"]) for r in _csv_rows([calib], "_counter_collection.csv")
                        if r["Counter_Name"] == cname and "copyBuffer" in r["Kernel_Name"]]
                if vals:
                    scale[cname] = 1048576.0 / (sum(vals) / len(vals))  # 1 GiB read and written
            out.append(f"HBM byte scale from a plain 1 GiB copy: FETCH_SIZE x {scale['FETCH_SIZE']:.3f}, "
                       f"WRITE_SIZE x {scale['WRITE_SIZE']:.3f}")
        per = {}   # kernel -> dispatch -> {counter: value, 'ns': duration}
        for r in pmc:
            # the counter passes are separate runs of the same program, so a
            # dispatch id names the same launch in each of them
            d = per.setdefault(r["Kernel_Name"], {}).setdefault(int(r["Dispatch_Id"]), {})
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        out.append(f"counters per dispatch (mean over the dispatches of the last {timed} calls):")
        traffic = None
        main = max((k for k in per if not any(x in k for x in SETUP_KERNELS)),
                   key=lambda k: means.get(k, 0.0), default=None)
        for k, ds in sorted(per.items(), key=lambda kv: -means.get(kv[0], 0.0)):
            if any(x in k for x in SETUP_KERNELS) or len(ds) < timed:
                continue
            # one dict per dispatch, merged over the counter passes in dispatch order
            vals = list(ds.values())
            per_call = _per_call(len(vals), timed, warmup)
            cnames = sorted({c for v in vals for c in v if c != "ns"})
            last = {}
            for c in cnames:
                xs = [v[c] for v in vals if c in v]
                xs = xs[-timed * per_call:] if len(xs) >= timed * per_call else xs
                last[c] = sum(xs) / len(xs)
            out.append(f"  {_short(k)}")
            line = []
            if "GRBM_GUI_ACTIVE" in last:
                cyc = last["GRBM_GUI_ACTIVE"] / NUM_XCD
                busy = last.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
                if busy > 0:
                    line.append(f"MFMA busy {100 * busy / (cyc * NUM_SIMD):.1f} % "
                                f"(SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM_GUI_ACTIVE / 8 XCDs))")
                ns = [v["ns"] for v in vals if "GRBM_GUI_ACTIVE" in v]
                ns = ns[-timed * per_call:] if len(ns) >= timed * per_call else ns
                if sum(ns) / len(ns) > 2e5:   # (shorter dispatches: GRBM counts beyond them)
                    line.append(f"engine clock {cyc / (sum(ns) / len(ns)):.2f} GHz (GRBM_GUI_ACTIVE / "
                                f"8 XCDs over the dispatch)")
                for c, what in (("SQ_INSTS_VALU_MFMA_MOPS_F32", "fp32"), ("SQ_INSTS_VALU_MFMA_MOPS_F16", "fp16")):
                    if last.get(c, 0.0) > 0:
                        fl = last[c] * 512
                        line.append(f"{what} MFMA flops {fl:.4g} ({c} x 512) = "
                                    f"{fl / (sum(ns) / len(ns)) / 1e3:.1f} TFLOP/s over the profiled dispatch")
            if "SQ_LDS_IDX_ACTIVE" in last and "SQ_LDS_BANK_CONFLICT" in last:
                bc, act = last["SQ_LDS_BANK_CONFLICT"], last["SQ_LDS_IDX_ACTIVE"]
                line.append(f"LDS bank conflicts {bc:.4g} cycles = {bc / max(act, 1):.4f} of the "
                            f"{act:.4g} indexed-LDS cycles (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; "
                            f"direct buffer-to-LDS loads are not indexed operations)")
            if "TCC_HIT_sum" in last and "TCC_MISS_sum" in last:
                h, m = last["TCC_HIT_sum"], last["TCC_MISS_sum"]
                line.append(f"L2 hit {100 * h / max(h + m, 1):.1f} % ({h:.4g} hits, {m:.4g} misses)")
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                if c in last:
                    line.append(f"{c} {last[c]:.1f} KiB x {scale[c]:.3f} = {last[c] * scale[c] * 1024:.4g} B")
            if "FETCH_SIZE" in last and "WRITE_SIZE" in last:
                t = (last["FETCH_SIZE"] * scale["FETCH_SIZE"] + last["WRITE_SIZE"] * scale["WRITE_SIZE"]) * 1024
                line.append(f"HBM traffic per dispatch {t:.4g} B")
                if k == main:
                    traffic = t
            for c in cnames:
                if c not in ("GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F32",
                             "SQ_INSTS_VALU_MFMA_MOPS_F16", "TCC_HIT_sum", "TCC_MISS_sum", "FETCH_SIZE",
                             "WRITE_SIZE", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE"):
                    line.append(f"{c} {last[c]:.6g}")
            for x in line:
                out.append(f"    {x}")
        if traffic is not None:
            out.append(f"traffic_bytes_per_launch: {traffic:.4g}  ({_short(main)})")
    return "\n".join(out)


# ---------------------------------------------------------------------------
def main() -> int:
    args = parse_args()
    if args.summarize:
        cfg = None
        if args.mode.startswith("torch:") and "," not in args.mode:
            cfg = adhoc_torch_gemm(args.mode)
        elif args.mode not in ("full", "gemm", "configs", "copy", "list"):
            sys.path.insert(0, REPO)
            import __graft_entry__
            cfg = {c.name: c for c in configs(__graft_entry__.load_package())}.get(args.mode)
        text = summarize(args.summarize, args.calib, args.steps, cfg,
                         args.warmup if cfg is not None else None)
        if cfg is not None:
            root = os.path.dirname(os.path.normpath(args.summarize[0]))
            root = os.path.relpath(os.path.dirname(root), REPO) if os.path.isabs(root) else os.path.dirname(root)
            text = "\n".join(summary_header(cfg, args.steps, args.warmup, root)) + "\n" + text
        print(text)
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the GEMM-family path has no multi-GPU leg here.", file=sys.stderr)
        return 2

    import torch

    sys.path.insert(0, REPO)
    import __graft_entry__

    ck = __graft_entry__.load_package()
    cfgs = configs(ck)
    if args.mode == "list":
        print("\n".join(["gemm", "configs", "copy"] + [c.name for c in cfgs]))
        return 0
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    u = make_filler(ck, dev, stream)
    by_name = {c.name: c for c in cfgs}

    if args.mode == "copy":
        src = u((1 << 28,), 5)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy: 1 GiB read + 1 GiB write x3")
        return 0
    if args.mode.startswith("gemm:"):
        # a comma-separated list of gemm:MxNxK[:LAYOUT][@OVERRIDE]; --override
        # applies where a spec names none
        for spec in args.mode.split(","):
            spec, _, ov = spec.partition("@")
            override = int(ov, 0) if ov else args.override
            c = adhoc_gemm(ck, spec, override)
            rc, plan = ck.abi.plan(c.M, c.N, c.K, op_a=c.op_a, op_b=c.op_b, workspace_bytes=1 << 40,
                                   plan_override=override)
            ck.abi.check(rc, "mi_gemm_plan")
            r = run_config(c, u, stream, reps=args.steps, warmup=args.warmup, exact_warmup=True)
            print(json.dumps({"config": spec, "override": hex(override), "plan": plan.plan_id,
                              "split_k": plan.split_k, "stream_k": plan.stream_k,
                              "sk_phases": plan.sk_phases, **r}), flush=True)
        return 0
    if args.mode.startswith("torch:"):
        for spec in args.mode.split(","):
            c = adhoc_torch_gemm(spec)
            r = run_config(c, u, stream, reps=args.steps, warmup=args.warmup, exact_warmup=True)
            print(json.dumps({"config": spec, "operator": "torch A @ B", **r}), flush=True)
        return 0
    if args.mode in by_name:
        c = by_name[args.mode]
        r = run_config(c, u, stream, reps=args.steps, warmup=args.warmup, exact_warmup=True)
        print(json.dumps({"config": c.name, **r}), flush=True)
        return 0
    if args.mode not in ("full", "gemm", "configs"):
        print(f"unknown --mode {args.mode}; see --mode list", file=sys.stderr)
        return 2

    out = {}
    if args.mode in ("full", "gemm"):
        out["gemm"], out["roofline"] = run_headline(ck, u, stream, args.steps, args.warmup)
    cpu = not args.no_cpu and args.mode == "full"
    if args.mode in ("full", "configs") and not args.no_configs:
        res = {}
        table = [c for c in cfgs
                 if not (args.mode == "full" and c.name.startswith("gemm_") and c.name.endswith("_8192"))]
        # (the headline step times the four 8192^3 layouts, cpu_baseline their host step)
        for c in table:
            res[c.name] = run_config(c, u, stream)
            log(f"config {c.name}: {res[c.name]}")
        if cpu:   # every host leg after every GPU timing
            torch.set_num_threads(os.cpu_count() or 1)
            for c in table:
                res[c.name]["cpu"] = run_cpu_leg(c, u)
                res[c.name]["gpu_over_cpu"] = round(res[c.name]["cpu"]["ms"] / res[c.name]["ms"], 1)
                log(f"cpu {c.name}: {res[c.name]['cpu']}")
        out["configs"] = res
    if args.mode != "full":
        if args.mode == "gemm":
            print(json.dumps(out["gemm"]), flush=True)
        return 0
    if args.no_configs and "configs" not in out:
        out["configs"] = None
    gemv = (out.get("configs") or {}).get("gemv_32768x65536")
    cpu_base = None
    if cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        cpu_base = cpu_headline(u)
        log(f"cpu baseline: {cpu_base['value']:.3f} TFLOP/s on {cpu_base['cores']} threads")

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
        "gemv": ({"shape": [GEMV_M, GEMV_K], "ms": gemv["ms"], "gbps": gemv["gbps"],
                  "frac": gemv["frac_hbm"], "algorithmic_bytes": 4 * (GEMV_M * GEMV_K + GEMV_K + GEMV_M),
                  "cpu": gemv.get("cpu")} if gemv else None),
        "configs": out.get("configs"),
        "cpu_baseline": cpu_base,
        "host": host_info() if cpu else None,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
