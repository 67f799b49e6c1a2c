"""GPU tests of the drop-in operator layer: each reference function name
(``ck.pNN.<name>(A, B)``, kernels/N_...) on torch tensors, against the fp64
oracle, including transposed-view inputs and the reference's zero-size paths."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, to_dev, to_host

pytestmark = pytest.mark.gpu


def _u(orc, shape, seed):
    return orc.uniform(shape, seed)


def test_every_pid_module(ck, orc, dev):
    M, K, N = 130, 96, 70
    a, b = _u(orc, (M, K), 1), _u(orc, (K, N), 2)
    A, B = to_dev(a), to_dev(b)
    ref = orc.gemm(a, b)
    for fn in (ck.p02.matmul_cuda, ck.p06.matmul_cuda, ck.p07.gemm_cuda, ck.p08.matmul_cuda):
        assert_close(orc, to_host(fn(A, B)), ref, K, what=str(fn))

    s = _u(orc, (N, N), 3)
    S = to_dev(s)
    assert_close(orc, to_host(ck.p01.matmul_cuda(S, S)), orc.gemm(s, s), N, what="p01")

    a3, b3 = _u(orc, (3, 20, 30), 4), _u(orc, (3, 30, 40), 5)
    assert_close(orc, to_host(ck.p03.batched_matmul_cuda(to_dev(a3), to_dev(b3))),
                 orc.gemm(a3, b3), 30, what="p03")

    x = _u(orc, (K, 1), 6)
    y = ck.p04.gemv_cuda(A, to_dev(x))
    assert tuple(y.shape) == (M, 1)
    assert_close(orc, to_host(y)[:, 0], orc.gemv(a, x[:, 0]), K, what="p04")

    ts_a, ts_b = _u(orc, (200, 16), 7), _u(orc, (16, 200), 8)
    assert_close(orc, to_host(ck.p09.tall_skinny_matmul_cuda(to_dev(ts_a), to_dev(ts_b))),
                 orc.gemm(ts_a, ts_b), 16, what="p09")

    t3, w = _u(orc, (4, 25, K), 9), _u(orc, (K, N), 10)
    out = ck.p10.batched_matmul_cuda(to_dev(t3), to_dev(w))
    assert tuple(out.shape) == (4, 25, N)
    assert_close(orc, to_host(out).reshape(-1, N), orc.gemm(t3.reshape(-1, K), w), K, what="p10")

    t4 = _u(orc, (2, 3, 5, K), 11)
    out = ck.p11.tensor_matmul_cuda(to_dev(t4), to_dev(w))
    assert tuple(out.shape) == (2, 3, 5, N)
    assert_close(orc, to_host(out).reshape(-1, N), orc.gemm(t4.reshape(-1, K), w), K, what="p11")

    d = _u(orc, (M,), 12)
    np.testing.assert_array_equal(to_host(ck.p12.diag_mult_cuda(to_dev(d), A)), orc.diag_mult(d, a))

    r1, r2 = _u(orc, (N, N), 13), _u(orc, (N, N), 14)
    sa, sb = (r1 + r1.T) / 2, (r2 + r2.T) / 2
    assert_close(orc, to_host(ck.p13.symmetric_matmul_cuda(to_dev(sa), to_dev(sb))),
                 orc.gemm(sa, sb), N, what="p13")
    up = to_host(ck.p14.upper_tri_matmul_cuda(to_dev(np.triu(r1)), to_dev(np.triu(r2))))
    assert_close(orc, up, orc.gemm(np.triu(r1), np.triu(r2), orc.UPPER), N, what="p14")
    lo = to_host(ck.p15.lower_tri_mul_cuda(to_dev(np.tril(r1)), to_dev(np.tril(r2))))
    assert_close(orc, lo, orc.gemm(np.tril(r1), np.tril(r2), orc.LOWER), N, what="p15")

    at, bt = _u(orc, (K, M), 15), _u(orc, (N, K), 16)
    assert_close(orc, to_host(ck.p16.matmul_transposed_cuda(to_dev(at), B)),
                 orc.gemm(at.T, b), K, what="p16")
    assert_close(orc, to_host(ck.p17.matmul_cuda(A, to_dev(bt))), orc.gemm(a, bt.T), K,
                 what="p17")
    assert_close(orc, to_host(ck.p18.matmul_transposed_cuda(to_dev(at), to_dev(bt))),
                 orc.gemm(at.T, bt.T), K, what="p18")


def test_transposed_views_are_consumed_in_place(ck, orc, dev):
    M, K, N = 100, 80, 60
    a, b = _u(orc, (K, M), 21), _u(orc, (N, K), 22)  # stored transposed
    A_view, B_view = to_dev(a).t(), to_dev(b).t()     # logical M x K and K x N views
    assert not A_view.is_contiguous() and not B_view.is_contiguous()
    got = to_host(ck.p02.matmul_cuda(A_view, B_view))
    assert_close(orc, got, orc.gemm(a.T, b.T), K, what="views")
    # a sliced (non-unit, non-transposed) view goes through a copy
    big = to_dev(_u(orc, (M, 2 * K), 23))
    sl = big[:, ::2]
    got = to_host(ck.p02.matmul_cuda(sl, to_dev(b.T.copy())))
    assert_close(orc, got, orc.gemm(np.ascontiguousarray(to_host(sl)), b.T.copy()), K, what="slice")


def test_model_new_wrappers(ck, orc, dev):
    a, b = _u(orc, (64, 48), 31), _u(orc, (48, 32), 32)
    out = ck.ModelNew(2)(to_dev(a), to_dev(b))
    assert_close(orc, to_host(out), orc.gemm(a, b), 48, what="ModelNew(2)")
    with pytest.raises(ValueError):
        ck.ModelNew(98)


def test_zero_size_inputs(ck, dev):
    e = torch.empty((0, 5), device="cuda")
    f = torch.empty((5, 3), device="cuda")
    assert tuple(ck.p02.matmul_cuda(e, f).shape) == (0, 3)
    z = ck.p02.matmul_cuda(torch.empty((4, 0), device="cuda"), torch.empty((0, 3), device="cuda"))
    assert tuple(z.shape) == (4, 3) and torch.all(z == 0)
    assert tuple(ck.p01.matmul_cuda(torch.empty((0, 0), device="cuda"),
                                    torch.empty((0, 0), device="cuda")).shape) == (0, 0)
    y = ck.p04.gemv_cuda(torch.empty((3, 0), device="cuda"), torch.empty((0, 1), device="cuda"))
    assert torch.all(y == 0)


def test_runs_on_current_stream(ck, orc, dev):
    a, b = _u(orc, (256, 256), 41), _u(orc, (256, 256), 42)
    A, B = to_dev(a), to_dev(b)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        C = ck.p02.matmul_cuda(A, B)
    s.synchronize()
    assert_close(orc, C.cpu().numpy(), orc.gemm(a, b), 256, what="side stream")


@pytest.mark.parametrize("M,K,N,cfg,split", [(300, 5000, 300, 1, 16), (512, 2048, 512, 10, 4),
                                             (1024, 1024, 1024, 10, 1), (256, 4096, 256, 10, 16),
                                             (768, 3072, 768, 10, 1)])
def test_small_deep_products_split_by_default(ck, orc, dev, M, K, N, cfg, split):
    """Problems whose 128 / 256 tiles would leave most CUs idle take small
    tiles by default -- the 64-tile k-split config where K is a multiple of
    64 -- split along K where those still do not fill the CUs, with the
    workspace from the caching allocator; the fixed-order reductions (the
    waves' partial tiles, the splits) keep repeated calls bitwise equal."""
    rc, p = ck.abi.plan(M, N, K, workspace_bytes=1 << 40)
    assert rc == 0 and (p.plan_id, p.split_k) == (cfg, split), (M, N, K, p.plan_id, p.split_k)
    a, b = _u(orc, (M, K), 91), _u(orc, (K, N), 92)
    A, B = to_dev(a), to_dev(b)
    C1 = ck.p02.matmul_cuda(A, B)
    C2 = ck.p02.matmul_cuda(A, B)
    assert torch.equal(C1, C2)
    assert_close(orc, to_host(C1), orc.gemm(a, b), K, what=f"split by default {M}x{K}x{N}")


def test_operators_replay_in_a_hip_graph(ck, dev):
    """The operators only launch kernels on the current stream (no host
    synchronisation, no memset; workspaces from the caching allocator), so a
    sequence of them can be captured in a HIP graph: captured once, replayed
    three times with eager work and synchronisations between the replays,
    every replay bitwise equal to the eager results.  Covers the direct-staged
    256 and 128 tiles, split-K with its reduction (workspace), stream-K with
    its fixup on the 256 and 32-deep 128 tiles, the 32-deep tile data-parallel
    and split, the 64-tile k-split config alone and split, the chunked
    triangular list with its finishing pass, GEMV,
    diag, pointwise conv and attention."""
    g = torch.Generator(device="cuda")
    g.manual_seed(97)
    u = lambda *shape: torch.rand(*shape, device="cuda", generator=g) * 2 - 1
    a4, b4 = u(4096, 4096), u(4096, 4096)
    a2, b2 = u(2048, 768), u(768, 1536)
    lka, lkb = u(256, 1 << 17), u(1 << 17, 256)
    ta, tb = u(6144, 6144).tril_(), u(6144, 6144).tril_()
    ga, gx = u(4096, 8192), u(8192, 1)
    dv, dm = u(2048), u(2048, 2048)
    cx, cw, cb = u(2, 64, 64, 64), u(128, 64), u(128)
    q, k, v = (u(1, 2, 128, 1024).half() for _ in range(3))
    # plans: stream-K on the 256 tile, stream-K / split-K on the 32-deep 128
    # tile, data-parallel on the 8-wave 128 tile (asserted below)
    sk3a, sk3b = u(3072, 12288), u(12288, 3072)
    sk9a, sk9b = u(1280, 8192), u(8192, 1280)
    d9a, d9b = u(2048, 2048), u(2048, 4096)
    s9a, s9b = u(1024, 8192), u(8192, 2048)
    # ... and the 64-tile k-split config, alone and split
    k10a, k10b = u(1024, 1024), u(1024, 1024)
    k10sa, k10sb = u(512, 8192), u(8192, 512)
    for (m, kk, n), want in [((3072, 12288, 3072), (3, 1, 1)), ((1280, 8192, 1280), (9, 1, 1)),
                             ((2048, 2048, 4096), (11, 0, 1)), ((1024, 8192, 2048), (9, 0, 4)),
                             ((1024, 1024, 1024), (10, 0, 1)), ((512, 8192, 512), (10, 0, 4))]:
        rc, p = ck.abi.plan(m, n, kk, workspace_bytes=1 << 40)
        assert rc == 0 and (p.plan_id, p.stream_k, p.split_k) == want, (m, kk, n, p.plan_id, p.stream_k,
                                                                         p.split_k)

    def ops():
        return [ck.p02.matmul_cuda(sk3a, sk3b), ck.p02.matmul_cuda(sk9a, sk9b), ck.p02.matmul_cuda(d9a, d9b),
                ck.p02.matmul_cuda(s9a, s9b), ck.p01.matmul_cuda(k10a, k10b), ck.p02.matmul_cuda(k10sa, k10sb),
                ck.p01.matmul_cuda(a4, b4), ck.p02.matmul_cuda(a2, b2), ck.p06.matmul_cuda(lka, lkb),
                ck.p15.lower_tri_mul_cuda(ta, tb), ck.p04.gemv_cuda(ga, gx), ck.p12.diag_mult_cuda(dv, dm),
                ck.p87.pointwise_conv_cuda(cx, cw, cb), ck.p97.fused_attention_cuda(q, k, v)]

    eager = [x.clone() for x in ops()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream
        ops()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = ops()
    for rep in range(3):
        for o in outs:  # eager work between replays
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep}: operator {i} differs from its eager result"


def test_operators_reentrant_across_threads_and_streams(ck, dev):
    """No global mutable state: four host threads, each on its own stream,
    run different operators concurrently (split-K workspaces from the caching
    allocator, the triangular list's finishing pass, attention's workspace);
    every result bitwise equals the same call made alone."""
    import threading

    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    u = lambda *shape: torch.rand(*shape, device="cuda", generator=g) * 2 - 1
    jobs = [
        (lambda x, y: ck.p06.matmul_cuda(x, y), (u(256, 1 << 16), u(1 << 16, 256))),
        (lambda x, y: ck.p14.upper_tri_matmul_cuda(x, y), (u(6144, 6144).triu_(), u(6144, 6144).triu_())),
        (lambda x, y: ck.p16.matmul_transposed_cuda(x, y), (u(1024, 2048), u(1024, 3000))),
        (lambda x, y: ck.p97.fused_attention_cuda(x, y, y), (u(1, 4, 256, 1024).half(), u(1, 4, 256, 1024).half())),
    ]
    alone = [fn(*args).clone() for fn, args in jobs]
    torch.cuda.synchronize()
    results, errors = [None] * len(jobs), []

    def run(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [jobs[i][0](*jobs[i][1]) for _ in range(3)]
            s.synchronize()
            results[i] = outs
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, outs in enumerate(results):
        for o in outs:
            assert torch.equal(o, alone[i]), f"job {i} differs when run concurrently"


def test_matrix_scalar_operator(ck, orc, dev):
    """PID 5 matrix_scalar_mult_cuda(A, float s) (kernels/5_...:47-71): the
    output is empty_like(A) (any shape), bitwise the fp32 product, an empty A
    returns an empty C, and the reference's three checks."""
    a = _u(orc, (3, 50, 71), 30)
    A = to_dev(a)
    for fn in (lambda x: ck.p05.matrix_scalar_mult_cuda(x, 3.14),
               lambda x: ck.ModelNew(5)(x, 3.14), lambda x: ck.ModelNew(5)(x, torch.tensor(3.14))):
        C = fn(A)
        assert C.shape == A.shape and C.dtype == torch.float32
        np.testing.assert_array_equal(to_host(C).view(np.uint32), orc.scale(a, 3.14).view(np.uint32))
    e = ck.p05.matrix_scalar_mult_cuda(torch.empty((0, 5), device="cuda"), 2.0)
    assert tuple(e.shape) == (0, 5)
    with pytest.raises(RuntimeError, match="A must be float32"):
        ck.p05.matrix_scalar_mult_cuda(A.double(), 2.0)
    with pytest.raises(RuntimeError, match="A must be contiguous"):
        ck.p05.matrix_scalar_mult_cuda(A.transpose(1, 2), 2.0)


@pytest.mark.parametrize("n,cin,cout,h,w,with_bias", [
    (2, 3, 64, 17, 17, True),      # K = 3: element-load path, odd H*W
    (4, 64, 128, 32, 32, True),    # single-slice K = 64
    (4, 64, 128, 32, 32, False),
    (1, 256, 96, 40, 40, True),    # several K slices
    (2, 32, 2048, 64, 64, True),   # M = 2048: the A-panel kernel
    (3, 0, 8, 5, 5, True),         # no input channels: out = bias
    (3, 0, 8, 5, 5, False),        # ... or zeros
])
def test_pointwise_conv_operator(ck, orc, dev, n, cin, cout, h, w, with_bias):
    """PID 87 pointwise_conv_cuda(input, weight, bias) (kernels/87_...:451-492)
    against the fp64 oracle: output N x Cout x H x W, bias added once."""
    x = _u(orc, (n, cin, h, w), 40)
    wt = _u(orc, (cout, cin, 1, 1), 41)
    b = _u(orc, (cout,), 42) if with_bias else None
    out = ck.p87.pointwise_conv_cuda(to_dev(x), to_dev(wt), None if b is None else to_dev(b))
    assert tuple(out.shape) == (n, cout, h, w)
    ref = orc.pointwise_conv(x, wt, b)
    if cin == 0:
        np.testing.assert_array_equal(to_host(out), ref.astype(np.float32))
    else:
        assert_close(orc, to_host(out).reshape(-1), ref.reshape(-1), cin,
                     what=f"conv {n}x{cin}x{cout}x{h}x{w} bias={with_bias}")
    # ModelNew(87) and a 2-D weight give the same result
    again = ck.ModelNew(87)(to_dev(x), to_dev(wt[:, :, 0, 0]), None if b is None else to_dev(b))
    np.testing.assert_array_equal(to_host(again), to_host(out))


def test_pointwise_conv_empty_and_checks(ck, dev):
    out = ck.p87.pointwise_conv_cuda(torch.empty((0, 4, 3, 3), device="cuda"),
                                     torch.empty((5, 4, 1, 1), device="cuda"))
    assert tuple(out.shape) == (0, 5, 3, 3)
    x = torch.zeros((1, 4, 3, 3), device="cuda")
    with pytest.raises(RuntimeError, match="weight.size"):
        ck.p87.pointwise_conv_cuda(x, torch.zeros((5, 3), device="cuda"))
    with pytest.raises(RuntimeError, match="bias must have C_out"):
        ck.p87.pointwise_conv_cuda(x, torch.zeros((5, 4), device="cuda"), torch.zeros(4, device="cuda"))
    with pytest.raises(RuntimeError, match="float32"):
        ck.p87.pointwise_conv_cuda(x.double(), torch.zeros((5, 4), device="cuda", dtype=torch.float64))


@pytest.mark.parametrize("M,K,N,ta,tb", [(1030, 517, 1027, False, False), (513, 1031, 770, True, False),
                                         (600, 401, 999, False, True), (515, 1029, 515, True, True)])
def test_unaligned_rows_in_place(ck, orc, dev, M, K, N, ta, tb):
    """Large products whose rows are not 16-byte aligned (kernels/8_... style
    irregular extents) run on the operands in place (4-byte direct staging,
    partial last K slice); results and the output shape are those of the
    plain product."""
    a_st = _u(orc, (K, M) if ta else (M, K), 70)
    b_st = _u(orc, (N, K) if tb else (K, N), 71)
    A = to_dev(a_st).t() if ta else to_dev(a_st)
    B = to_dev(b_st).t() if tb else to_dev(b_st)
    C = ck.p08.matmul_cuda(A, B)
    assert tuple(C.shape) == (M, N) and C.is_contiguous()
    ref = orc.gemm(a_st.T if ta else a_st, b_st.T if tb else b_st)
    assert_close(orc, to_host(C), ref, K, what=f"unaligned {M}x{K}x{N} {ta}{tb}")


def test_torch_ops_dispatch_to_the_kernels(ck, orc, dev):
    """torch.ops.mi355.<op> runs the same HIP kernels as the per-PID modules."""
    a, b = _u(orc, (130, 96), 80), _u(orc, (96, 70), 81)
    A, B = to_dev(a), to_dev(b)
    np.testing.assert_array_equal(to_host(torch.ops.mi355.matmul(A, B)), to_host(ck.p02.matmul_cuda(A, B)))
    np.testing.assert_array_equal(to_host(torch.ops.mi355.matrix_scalar_mult(A, 2.5)),
                                  to_host(ck.p05.matrix_scalar_mult_cuda(A, 2.5)))
    d = to_dev(_u(orc, (130,), 82))
    np.testing.assert_array_equal(to_host(torch.ops.mi355.diag_mult(d, A)), to_host(ck.p12.diag_mult_cuda(d, A)))


def test_golden_fixtures_bitwise(ck, dev):
    """Every operator on the committed integer known-answer cases
    (tests/golden/gemm_family_int.npz): exact arithmetic, so bitwise equal."""
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemm_family_int.npz"))
    names = sorted({k.split(".")[0] for k in z.files})
    fn = {
        "p01_square": ck.p01.matmul_cuda, "p02_matmul": ck.p02.matmul_cuda,
        "p03_batched": ck.p03.batched_matmul_cuda, "p04_gemv": ck.p04.gemv_cuda,
        "p06_large_k": ck.p06.matmul_cuda, "p07_small_k": ck.p07.gemm_cuda,
        "p08_irregular": ck.p08.matmul_cuda, "p09_tall_skinny": ck.p09.tall_skinny_matmul_cuda,
        "p10_tensor3d": ck.p10.batched_matmul_cuda, "p11_tensor4d": ck.p11.tensor_matmul_cuda,
        "p12_diag": ck.p12.diag_mult_cuda, "p13_symmetric": ck.p13.symmetric_matmul_cuda,
        "p14_upper": ck.p14.upper_tri_matmul_cuda, "p15_lower": ck.p15.lower_tri_mul_cuda,
        "p16_transposed_a": ck.p16.matmul_transposed_cuda, "p17_transposed_b": ck.p17.matmul_cuda,
        "p18_transposed_both": ck.p18.matmul_transposed_cuda,
        "p05_scalar": lambda A, B: ck.p05.matrix_scalar_mult_cuda(A, float(B[0])),
        "p87_pointwise": lambda A, B: ck.p87.pointwise_conv_cuda(
            A, B, to_dev(z["p87_pointwise.bias"])),
    }
    assert set(fn) == set(names)
    for name in names:
        A, B, C = z[f"{name}.A"], z[f"{name}.B"], z[f"{name}.C"]
        got = to_host(fn[name](to_dev(A), to_dev(B)))
        np.testing.assert_array_equal(got, C, err_msg=name)
