"""CPU tests of the drop-in operator layer's error behaviour: every check fires
before any launch, with the reference's TORCH_CHECK message where the
reference has one (file:line in each case), surfacing as RuntimeError."""
import pytest
import torch


def _f(*shape):
    return torch.zeros(shape, dtype=torch.float32)


CASES = [
    # (pid submodule, function, A, B, expected message fragment)
    ("p02", "matmul_cuda", _f(3), _f(3, 3), "A must be 2D"),                 # kernels/2_...:118
    ("p02", "matmul_cuda", _f(3, 4), _f(3, 4), "Matrix dimensions do not match"),  # 2_...:120
    ("p03", "batched_matmul_cuda", _f(2, 3), _f(2, 3, 4), "A must be 3D tensor"),  # 3_...:114
    ("p03", "batched_matmul_cuda", _f(2, 3, 4), _f(3, 4), "B must be 3D tensor"),  # 3_...:115
    ("p04", "gemv_cuda", _f(3), _f(3, 1), "A must be 2D"),                   # 4_...:85
    ("p04", "gemv_cuda", _f(3, 4), _f(5, 1), "A and B shapes not matched"),  # 4_...:89
    ("p04", "gemv_cuda", _f(3, 4), _f(4, 2), "B must be a column vector"),  # 4_...:90
    ("p06", "matmul_cuda", _f(3, 4), _f(5, 6), "Matrix dimensions mismatch"),  # 6_...:133
    ("p12", "diag_mult_cuda", _f(4), _f(4, 5), "A must be a CUDA tensor"),   # 12_...:44
    ("p14", "upper_tri_matmul_cuda", _f(3, 4), _f(4, 4), "A must be square"),  # 14_...:138
    ("p14", "upper_tri_matmul_cuda", _f(4, 4), _f(5, 5), "A and B must have the same size"),
    ("p15", "lower_tri_mul_cuda", _f(4, 4), _f(3, 4), "B must have the same size as A"),
    ("p15", "lower_tri_mul_cuda", _f(4, 4), _f(4, 3), "B must be square"),   # 15_...:161
    ("p15", "lower_tri_mul_cuda", _f(4, 4), _f(4, 4), "A must be on CUDA"),  # 15_...:162
    ("p16", "matmul_transposed_cuda", _f(3, 4), _f(5, 4),
     "A and B must have the same number of rows"),                          # 16_...:130
]


@pytest.mark.parametrize("A,msg", [
    (_f(4, 4), "A must be a CUDA tensor"),                                  # 5_...:48
])
def test_matrix_scalar_messages(ck, A, msg):
    with pytest.raises(RuntimeError, match=msg):
        ck.p05.matrix_scalar_mult_cuda(A, 2.0)
    with pytest.raises(RuntimeError, match=msg):
        ck.ModelNew(5)(A, 2.0)


@pytest.mark.parametrize("x,w,b,msg", [
    (_f(2, 3, 4), _f(5, 3), None, "input must be 4D"),
    (_f(2, 3, 4, 4), _f(5, 3, 3, 3), None, "weight must be"),
    (_f(2, 3, 4, 4), _f(5, 3, 1, 1), None, "input must be a CUDA tensor"),
])
def test_pointwise_conv_checks(ck, x, w, b, msg):
    with pytest.raises(RuntimeError, match=msg):
        ck.p87.pointwise_conv_cuda(x, w, b)


def _h(*shape):
    return torch.zeros(shape, dtype=torch.float16)


@pytest.mark.parametrize("q,msg", [
    (_h(1, 1, 600, 1024), "Sequence length exceeds MAX_SEQ_LENGTH."),      # 97_...:267
    (_h(1, 1, 64, 512), "Embedding dimension must be 1024."),              # 97_...:268
    (_h(64, 1024), "must be 4D"),
    (_h(1, 1, 64, 1024), "CUDA tensors"),
])
def test_fused_attention_checks(ck, q, msg):
    with pytest.raises(RuntimeError, match=msg):
        ck.p97.fused_attention_cuda(q, q, q)


@pytest.mark.parametrize("sub,name,A,B,msg", CASES)
def test_reference_error_messages(ck, sub, name, A, B, msg):
    fn = getattr(getattr(ck, sub), name)
    with pytest.raises(RuntimeError, match=msg):
        fn(A, B)


@pytest.mark.parametrize("pid", [1, 2, 3, 6, 7, 8, 9, 10, 11, 13, 16, 17, 18])
def test_cpu_tensors_are_rejected_not_computed(ck, pid):
    # Shapes valid for every operator; the device check must refuse CPU
    # tensors instead of falling back to a CPU computation.
    shapes = {3: ((2, 4, 4), (2, 4, 4)), 10: ((2, 4, 4), (4, 4)), 11: ((1, 2, 2, 4), (4, 4))}
    sa, sb = shapes.get(pid, ((4, 4), (4, 4)))
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ck.ModelNew(pid)(_f(*sa), _f(*sb))


def test_dtype_is_checked(ck):
    a = torch.zeros((4, 4), dtype=torch.float64)
    with pytest.raises(RuntimeError, match="(CUDA tensor|float32)"):
        ck.p02.matmul_cuda(a, a)


def test_model_new_registry(ck):
    assert ck.PIDS == tuple(range(1, 19)) + (87, 97)
    for pid in ck.PIDS:
        m = ck.ModelNew(pid)
        assert isinstance(m, torch.nn.Module) and ck.OPS[pid][1] in repr(m)
    for pid in (0, 19, 86, 98):
        with pytest.raises(ValueError):
            ck.ModelNew(pid)


def test_package_refuses_to_load_without_extension(tmp_path):
    # A copy of the package directory without the built libraries must fail at
    # import instead of silently offering a non-native fallback.
    import importlib.util
    import shutil
    import sys
    import os
    src = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "cupilot-kernels_amd")
    dst = tmp_path / "pkg"
    shutil.copytree(src, dst, ignore=shutil.ignore_patterns("*.so", "_build", "csrc"))
    spec = importlib.util.spec_from_file_location("ck_nobuild", dst / "__init__.py",
                                                  submodule_search_locations=[str(dst)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ck_nobuild"] = mod
    try:
        with pytest.raises(ImportError, match="not built"):
            spec.loader.exec_module(mod)
    finally:
        sys.modules.pop("ck_nobuild", None)


def test_torch_ops_registered_with_meta_shapes(ck):
    """Every operator is also torch.ops.mi355.<op> (graph use): Meta kernels
    give the reference output shapes, and a CPU tensor is rejected (no CPU
    kernel, so no silent fallback)."""
    import torch
    ops = torch.ops.mi355
    m = lambda *s: torch.empty(s, device="meta")
    cases = {
        "square_matmul": ((m(8, 8), m(8, 8)), (8, 8)),
        "matmul": ((m(5, 7), m(7, 3)), (5, 3)),
        "batched_matmul": ((m(2, 5, 7), m(2, 7, 3)), (2, 5, 3)),
        "gemv": ((m(5, 7), m(7, 1)), (5, 1)),
        "matmul_large_k": ((m(4, 4096), m(4096, 6)), (4, 6)),
        "gemm_small_k": ((m(9, 2), m(2, 11)), (9, 11)),
        "tall_skinny_matmul": ((m(12, 3), m(3, 12)), (12, 12)),
        "tensor3d_matmul": ((m(2, 5, 7), m(7, 3)), (2, 5, 3)),
        "tensor4d_matmul": ((m(2, 3, 4, 7), m(7, 5)), (2, 3, 4, 5)),
        "diag_mult": ((m(6), m(6, 9)), (6, 9)),
        "symmetric_matmul": ((m(8, 8), m(8, 8)), (8, 8)),
        "upper_tri_matmul": ((m(8, 8), m(8, 8)), (8, 8)),
        "lower_tri_mul": ((m(8, 8), m(8, 8)), (8, 8)),
        "matmul_transposed_a": ((m(7, 5), m(7, 3)), (5, 3)),
        "matmul_transposed_b": ((m(5, 7), m(3, 7)), (5, 3)),
        "matmul_transposed_both": ((m(7, 5), m(3, 7)), (5, 3)),
        "fused_attention": ((m(1, 2, 16, 1024),) * 3, (1, 2, 16, 1024)),
    }
    for name, (args, shape) in cases.items():
        assert tuple(getattr(ops, name)(*args).shape) == shape, name
    assert tuple(ops.matrix_scalar_mult(m(3, 4), 2.0).shape) == (3, 4)
    assert tuple(ops.pointwise_conv(m(2, 3, 5, 5), m(8, 3, 1, 1), None).shape) == (2, 8, 5, 5)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.matmul(torch.zeros(4, 4), torch.zeros(4, 4))
