"""ctypes binding of the C ABI in include/mi355_gemm.h (libmi355gemm.so).

This is the binding a Python host would write against the library; the GPU
parity tests call the kernels through it, so what they check is the C
boundary itself.  torch must be imported before the library is loaded so that
the library binds to the HIP runtime torch already loaded (both carry the
soname libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmi355gemm.so")

MI_OK = 0
MI_ERR_NULL_POINTER = -1
MI_ERR_BAD_SIZE = -2
MI_ERR_BAD_LAYOUT = -3
MI_ERR_BAD_LD = -4
MI_ERR_NOT_SQUARE = -5
MI_ERR_WORKSPACE = -6
MI_ERR_NO_DEVICE = -7
MI_ERR_ALIGNMENT = -8
MI_ERR_SCRATCH_LIMIT = -9
NOALLOC_SCRATCH_BYTES = 64 << 20

MI_OP_N, MI_OP_T = 0, 1
MI_DENSE, MI_LOWER, MI_UPPER, MI_SYMMETRIC = 0, 1, 2, 3
(CFG64, CFG128, CFG256, CFG128K32, CFG128K64, CFG_PANEL32, CFG_PANEL64, CFG_PANEL128, CFG128B32,
 CFG64W, CFG128W8, CFG_PANEL64B) = (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12)
PLAN_NO_PACK, PLAN_PACK = 0x40, 0x80  # plan_override bits (operand packing)

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t


class GemmArgs(ctypes.Structure):
    """mirror of mi_gemm_args"""
    _fields_ = [
        ("A", _vp), ("B", _vp), ("C", _vp),
        ("M", _i64), ("N", _i64), ("K", _i64), ("batch", _i64),
        ("lda", _i64), ("ldb", _i64), ("ldc", _i64),
        ("stride_a", _i64), ("stride_b", _i64), ("stride_c", _i64),
        ("op_a", ctypes.c_int32), ("op_b", ctypes.c_int32),
        ("structure", ctypes.c_int32), ("plan_override", ctypes.c_int32),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("bias_m", _vp),
    ]


class Plan(ctypes.Structure):
    """mirror of mi_plan"""
    _fields_ = [
        ("plan_id", ctypes.c_int32), ("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32),
        ("block_k", ctypes.c_int32), ("tiles_m", ctypes.c_int32), ("tiles_n", ctypes.c_int32),
        ("split_k", ctypes.c_int32), ("k_chunk", _i64), ("group_m", ctypes.c_int32),
        ("num_tiles", _i64), ("grid", _i64), ("workspace_bytes", _sz),
        ("stream_k", ctypes.c_int32), ("sk_tiles", _i64),
        ("packed", ctypes.c_int32), ("packed_k", _i64), ("sk_phases", ctypes.c_int32),
    ]


class WorkItem(ctypes.Structure):
    """mirror of mi_work_item"""
    _fields_ = [
        ("tile_m", ctypes.c_int32), ("tile_n", ctypes.c_int32),
        ("k_begin", _i64), ("k_end", _i64), ("dest", ctypes.c_int32), ("slot", ctypes.c_int32),
    ]


# name -> (restype, argtypes); every symbol include/mi355_gemm.h declares
SIGNATURES = {
    "mi_gemm_f32": (ctypes.c_int, [ctypes.POINTER(GemmArgs), _vp]),
    "mi_gemm_f32_noalloc": (ctypes.c_int, [ctypes.POINTER(GemmArgs), _vp]),
    "mi_gemm_work_item": (ctypes.c_int, [ctypes.POINTER(GemmArgs), ctypes.c_int32, _i64, ctypes.c_int32,
                                         _i64, ctypes.POINTER(WorkItem)]),
    "mi_gemm_sk_fixup_of": (ctypes.c_int, [ctypes.POINTER(GemmArgs), ctypes.c_int32, _i64,
                                           ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "mi_gemm_workspace_bytes": (_sz, [ctypes.POINTER(GemmArgs)]),
    "mi_gemm_plan": (ctypes.c_int, [ctypes.POINTER(GemmArgs), ctypes.c_int32, ctypes.POINTER(Plan)]),
    "mi_gemm_tile_of": (ctypes.c_int, [ctypes.POINTER(GemmArgs), ctypes.c_int32, _i64, ctypes.c_int32,
                                       ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                       ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "mi_square_matmul_workspace_bytes": (_sz, [_i64]),
    "mi_square_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "mi_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_batched_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "mi_batched_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_gemv_workspace_bytes": (_sz, [_i64, _i64]),
    "mi_gemv_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _vp, _sz, _vp]),
    "mi_matmul_large_k_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_matmul_large_k_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_gemm_small_k_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "mi_tall_skinny_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "mi_tensor3d_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "mi_tensor3d_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_tensor4d_matmul_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "mi_tensor4d_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_diag_mult_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "mi_matrix_scalar_mult_f32": (ctypes.c_int, [_vp, _vp, _i64, ctypes.c_float, _vp]),
    "mi_pointwise_conv_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "mi_sdpa_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_sdpa_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_symmetric_matmul_workspace_bytes": (_sz, [_i64]),
    "mi_symmetric_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "mi_upper_tri_matmul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp]),
    "mi_lower_tri_mul_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp]),
    "mi_matmul_transposed_a_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_matmul_transposed_a_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_matmul_transposed_b_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_matmul_transposed_b_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_matmul_transposed_both_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "mi_matmul_transposed_both_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "mi_fill_uniform_f32": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64, _i64, _vp]),
    "mi_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mi_version": (ctypes.c_char_p, []),
}

_lib = None


def lib():
    """Load libmi355gemm.so (after torch) and attach the C signatures."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  -- bind to torch's HIP runtime
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run cupilot-kernels_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class MiError(RuntimeError):
    def __init__(self, status: int, where: str = ""):
        self.status = status
        msg = lib().mi_status_string(status).decode()
        super().__init__(f"{where}: {msg} (status {status})" if where else msg)


def check(status: int, where: str = "") -> None:
    if status != MI_OK:
        raise MiError(status, where)


def make_args(M, N, K, batch=1, op_a=MI_OP_N, op_b=MI_OP_N, structure=MI_DENSE,
              workspace_bytes=0, plan_override=0, lda=None, ldb=None, ldc=None):
    """An mi_gemm_args with no pointers (for the host-only queries)."""
    a = GemmArgs()
    a.M, a.N, a.K, a.batch = M, N, K, batch
    a.op_a, a.op_b, a.structure = op_a, op_b, structure
    a.lda = lda if lda is not None else (K if op_a == MI_OP_N else M)
    a.ldb = ldb if ldb is not None else (N if op_b == MI_OP_N else K)
    a.ldc = ldc if ldc is not None else N
    a.workspace_bytes = workspace_bytes
    a.plan_override = plan_override
    return a


def plan(M, N, K, num_cus=256, **kw):
    """Host-only scheduler query (mi_gemm_plan); no device needed."""
    a = make_args(M, N, K, **kw)
    p = Plan()
    rc = lib().mi_gemm_plan(ctypes.byref(a), num_cus, ctypes.byref(p))
    return rc, p


def work_items(args, wg, split=0, num_cus=256):
    """Every work item of workgroup wg in run order (mi_gemm_work_item):
    [(tile_m, tile_n, k_begin, k_end, dest, slot), ...]."""
    out, item = [], 0
    w = WorkItem()
    while True:
        rc = lib().mi_gemm_work_item(ctypes.byref(args), num_cus, wg, split, item, ctypes.byref(w))
        if rc < 0:
            raise RuntimeError(f"mi_gemm_work_item: {rc}")
        if rc == 0:
            return out
        out.append((w.tile_m, w.tile_n, w.k_begin, w.k_end, w.dest, w.slot))
        item += 1


def sk_fixup_of(args, t, num_cus=256):
    """(status, tile_m, tile_n, first_slot, n_slots) of stream-K tile t."""
    tm, tn = ctypes.c_int32(), ctypes.c_int32()
    f, n = _i64(), _i64()
    rc = lib().mi_gemm_sk_fixup_of(ctypes.byref(args), num_cus, t, ctypes.byref(tm), ctypes.byref(tn),
                                   ctypes.byref(f), ctypes.byref(n))
    return rc, tm.value, tn.value, f.value, n.value


def tile_of(args, wg, split=0, num_cus=256):
    """(status, tile_m, tile_n, k_begin, k_end) of work item wg (mi_gemm_tile_of)."""
    tm, tn = ctypes.c_int32(), ctypes.c_int32()
    kb, ke = _i64(), _i64()
    rc = lib().mi_gemm_tile_of(ctypes.byref(args), num_cus, wg, split, ctypes.byref(tm),
                               ctypes.byref(tn), ctypes.byref(kb), ctypes.byref(ke))
    return rc, tm.value, tn.value, kb.value, ke.value
