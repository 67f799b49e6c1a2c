"""The named dense C entry points with their workspace (kernels/6_...:128-203
splits deep K over the machine; kernels/8_...:155-168 takes any extents):
given the size their *_workspace_bytes query returns, they run the plan the
ATen operators run (split-K, stream-K, packed operand copies), so their bits
equal the operators' bits, and they are checked against the fp64 oracle
through row and column checksums of the whole output.  Without a workspace
they fall back to plans that need none, still within tolerance."""
import statistics

import numpy as np
import pytest
import torch

import freivalds as fv
from gpu_util import cur_stream, dev_uniform, to_host, vp

pytestmark = pytest.mark.gpu


def _ws(n):
    return torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")


def _checksums(orc, got, a, b, K, seed, what):
    v, u = fv.signs(got.shape[1], seed), fv.signs(got.shape[0], seed + 1)
    ref_cv, ref_utc = fv.reference(orc, a, b, v, u)
    cv, utc = got.astype(np.float64) @ v, u @ got.astype(np.float64)
    fv.check(orc, cv, utc, ref_cv, ref_utc, K, 1.0, 1.0, what=what)


# (M, K, N, entry, plan feature the preferred workspace buys)
CASES = [
    (256, 1 << 20, 256, "matmul", "split"),          # BASELINE large-K: split-K over the CUs
    (3072, 8192, 3072, "matmul", "stream_k"),        # stream-K
    (8205, 2949, 5921, "matmul", "packed"),          # PID 8's extents: packed operands
    (3072, 8192, 3072, "transposed_a", "stream_k"),
    (3072, 8192, 3072, "transposed_b", "stream_k"),
    (3072, 8192, 3072, "transposed_both", "stream_k"),
    (4608, 4608, 4608, "square", "stream_k"),
    (4608, 4608, 4608, "symmetric", "stream_k"),
]


def _entry(ck, name):
    """(C entry, its workspace query, the ATen operator, op_a, op_b)"""
    L = ck.abi.lib()
    table = {
        "matmul": (L.mi_matmul_f32, L.mi_matmul_workspace_bytes, ck.p02.matmul_cuda, 0, 0),
        "transposed_a": (L.mi_matmul_transposed_a_f32, L.mi_matmul_transposed_a_workspace_bytes,
                         ck.p16.matmul_transposed_cuda, 1, 0),
        "transposed_b": (L.mi_matmul_transposed_b_f32, L.mi_matmul_transposed_b_workspace_bytes,
                         ck.p17.matmul_cuda, 0, 1),
        "transposed_both": (L.mi_matmul_transposed_both_f32,
                            L.mi_matmul_transposed_both_workspace_bytes,
                            ck.p18.matmul_transposed_cuda, 1, 1),
        "square": (L.mi_square_matmul_f32, L.mi_square_matmul_workspace_bytes, ck.p01.matmul_cuda, 0, 0),
        "symmetric": (L.mi_symmetric_matmul_f32, L.mi_symmetric_matmul_workspace_bytes,
                      ck.p13.symmetric_matmul_cuda, 0, 0),
    }
    return table[name]


@pytest.mark.parametrize("M,K,N,name,feature", CASES)
def test_named_entry_with_workspace_equals_operator(ck, orc, dev, M, K, N, name, feature):
    fn, query, op, op_a, op_b = _entry(ck, name)
    square = name in ("square", "symmetric")
    nws = query(N) if square else query(M, K, N)
    assert nws > 0
    rc, p = ck.abi.plan(M, N, K, op_a=op_a, op_b=op_b, workspace_bytes=1 << 40)
    assert rc == 0 and p.workspace_bytes == nws
    assert {"split": p.split_k > 1, "stream_k": p.stream_k == 1, "packed": p.packed == 1}[feature]
    a_st = (dev_uniform(ck, (K, M), 901) if op_a else dev_uniform(ck, (M, K), 901))
    b_st = (dev_uniform(ck, (N, K), 902) if op_b else dev_uniform(ck, (K, N), 902))
    if name == "symmetric":
        a_st = (a_st + a_st.T) * 0.5
        b_st = (b_st + b_st.T) * 0.5
    # the operators of PIDs 16-18 take the stored (transposed) tensors, as
    # the C entries do
    want = to_host(op(a_st, b_st))
    ws = _ws(nws)
    C = torch.full((M, N), float("nan"), device="cuda")
    args = (vp(a_st), vp(b_st), vp(C)) + ((N,) if square else (M, K, N))
    ck.abi.check(fn(*args, vp(ws), nws, cur_stream()), fn.__name__)
    got = to_host(C)
    np.testing.assert_array_equal(got, want)
    la, lb = to_host(a_st), to_host(b_st)
    _checksums(orc, got, la.T if op_a else la, lb.T if op_b else lb, K, 910, f"{name} {M}x{K}x{N}")
    # no workspace: a plan that needs none, within tolerance
    C0 = torch.full((M, N), float("nan"), device="cuda")
    args0 = (vp(a_st), vp(b_st), vp(C0)) + ((N,) if square else (M, K, N))
    ck.abi.check(fn(*args0, None, 0, cur_stream()), fn.__name__ + " without workspace")
    _checksums(orc, to_host(C0), la.T if op_a else la, lb.T if op_b else lb, K, 920,
               f"{name} {M}x{K}x{N} no workspace")


def test_large_k_entry_runs_near_the_operator(ck, dev):
    """mi_matmul_f32 with its workspace at 256 x 256 x 2^20 (the BASELINE
    large-K shape) runs within 1.2x of p06.matmul_cuda (the same split-K
    plan; without a workspace the plan has only 16 workgroups)."""
    L = ck.abi.lib()
    M, K, N = 256, 1 << 20, 256
    A, B = dev_uniform(ck, (M, K), 931), dev_uniform(ck, (K, N), 932)
    C = torch.empty((M, N), device="cuda")
    nws = L.mi_matmul_workspace_bytes(M, K, N)
    ws = _ws(nws)
    s = cur_stream()

    def c_entry():
        ck.abi.check(L.mi_matmul_f32(vp(A), vp(B), vp(C), M, K, N, vp(ws), nws, s))

    def aten():
        ck.p06.matmul_cuda(A, B)

    times = {c_entry: [], aten: []}
    for f in (c_entry, aten):
        for _ in range(3):
            f()
    torch.cuda.synchronize()
    for _ in range(5):
        for f in (c_entry, aten):
            e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
            e0.record()
            for _ in range(5):
                f()
            e1.record()
            torch.cuda.synchronize()
            times[f].append(e0.elapsed_time(e1) / 5)
    t_c, t_a = statistics.median(times[c_entry]), statistics.median(times[aten])
    assert t_c <= 1.2 * t_a, f"C entry {t_c:.3f} ms vs operator {t_a:.3f} ms"
