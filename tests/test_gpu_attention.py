"""GPU parity of PID 97 scaled dot-product attention (kernels/97_...:136-296)
against the fp64 oracle: fp16 output within one binary16 spacing of the exact
result plus fp32-level error (the kernel keeps fp32-level error until its final
rounding, as the reference's fp32 arithmetic does), through
the operator (``ck.p97.fused_attention_cuda``), ``ModelNew(97)`` and the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import cur_stream, to_dev, to_host

pytestmark = pytest.mark.gpu


def _inputs(orc, shape, seed):
    return [orc.uniform(shape, seed + i).astype(np.float16) for i in range(3)]


def _check(orc, got, q, k, v, what):
    """|O - O64| <= one binary16 spacing of O64 + 2^-17 max|V|.  The spacing
    covers the final rounding to fp16; the absolute term covers fp32 rounding
    of the scores (accumulated in fp32, as the reference does), which exp()
    turns into a relative error of the weights of order |score| * 2^-24 * sqrt(E)
    -- visible only where the weighted sum cancels to a value far below max|V|
    (measured: 2.6e-6 at max|V| = 1, scores up to 19).  Dropping the low fp16
    term of the weights gives errors of ~4e-5 and fails this bound."""
    ref = orc.sdpa(q, k, v)
    err = np.abs(got.astype(np.float64) - ref)
    bound = orc.half_ulp(ref) + 2.0 ** -17 * float(np.max(np.abs(v.astype(np.float64))))
    worst = float(np.max(err / bound))
    assert worst <= 1.0, f"{what}: error {worst:.2f} x the bound"
    return worst


# (1, 130, 64, 1024) holds weights whose fp32 2^14 p falls exactly on an fp16
# rounding tie: an H / L split whose two roundings of H differ fails it.
@pytest.mark.parametrize("shape", [(1, 1, 512, 1024), (2, 3, 100, 1024), (1, 2, 1, 1024),
                                   (1, 1, 33, 1024), (1, 96, 512, 1024), (1, 130, 64, 1024),
                                   (2, 5, 300, 1024)])
def test_fused_attention_operator(ck, orc, dev, shape):
    q, k, v = _inputs(orc, shape, 40)
    Q, K, V = to_dev(q), to_dev(k), to_dev(v)
    out = ck.p97.fused_attention_cuda(Q, K, V)
    assert out.shape == Q.shape and out.dtype == torch.float16
    _check(orc, to_host(out), q, k, v, f"sdpa {shape}")
    again = ck.ModelNew(97)(Q, K, V)
    np.testing.assert_array_equal(to_host(again), to_host(out))


def test_fused_attention_large_scores(ck, orc, dev):
    """Scores far from zero (inputs scaled by 4: |s| up to ~500): the max
    subtraction keeps the softmax finite and the result within tolerance."""
    q, k, v = _inputs(orc, (1, 2, 256, 1024), 50)
    q = (q.astype(np.float32) * 4).astype(np.float16)
    k = (k.astype(np.float32) * 4).astype(np.float16)
    out = ck.p97.fused_attention_cuda(to_dev(q), to_dev(k), to_dev(v))
    _check(orc, to_host(out), q, k, v, "large scores")


def test_sdpa_abi_general_sizes_and_errors(ck, orc, dev):
    """The C entry point accepts any seq and embed % 64 == 0 (the operator
    keeps the reference's limits); it checks alignment, workspace and sizes."""
    L = ck.abi.lib()
    heads, seq, embed = 3, 200, 192
    q, k, v = _inputs(orc, (heads, seq, embed), 60)
    Q, K, V = to_dev(q), to_dev(k), to_dev(v)
    O = torch.empty_like(Q)
    nbytes = L.mi_sdpa_workspace_bytes(heads, seq, embed)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    vp = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off)
    ck.abi.check(L.mi_sdpa_f16(vp(Q), vp(K), vp(V), vp(O), heads, seq, embed, vp(ws), nbytes,
                               cur_stream()))
    _check(orc, to_host(O), q, k, v, "abi 3x200x192")
    assert L.mi_sdpa_f16(vp(Q), vp(K), vp(V), vp(O), heads, seq, embed, vp(ws), nbytes - 1,
                         cur_stream()) == ck.abi.MI_ERR_WORKSPACE
    assert L.mi_sdpa_f16(vp(Q, 2), vp(K), vp(V), vp(O), heads, seq, embed, vp(ws), nbytes,
                         cur_stream()) == ck.abi.MI_ERR_ALIGNMENT
    assert L.mi_sdpa_f16(vp(Q), vp(K), vp(V), vp(O), heads, seq, 100, vp(ws), nbytes,
                         cur_stream()) == ck.abi.MI_ERR_BAD_SIZE
    assert L.mi_sdpa_f16(None, None, None, None, 0, seq, embed, None, 0, cur_stream()) == 0


@pytest.mark.parametrize("heads,seq,embed", [(3, 512, 64), (2, 513, 64), (2, 700, 128), (1, 1100, 64)])
def test_sdpa_abi_kernel_paths(ck, orc, dev, heads, seq, embed):
    """Both schedules of the C entry point: seq <= 512 fuses the softmax into
    the QK kernel (here with a one-slice embed); longer rows keep fp32 scores
    in the workspace and split them with the register (seq <= 1024) or the
    three-pass row softmax, at and past the boundary."""
    L = ck.abi.lib()
    q, k, v = _inputs(orc, (heads, seq, embed), 70)
    Q, K, V = to_dev(q), to_dev(k), to_dev(v)
    O = torch.empty_like(Q)
    nbytes = L.mi_sdpa_workspace_bytes(heads, seq, embed)
    sp = -(-seq // 64) * 64
    assert nbytes == heads * (seq * 2 * sp * 2 + (0 if sp <= 512 else seq * sp * 4))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    ck.abi.check(L.mi_sdpa_f16(vp(Q), vp(K), vp(V), vp(O), heads, seq, embed, vp(ws), nbytes,
                               cur_stream()))
    _check(orc, to_host(O), q, k, v, f"abi {heads}x{seq}x{embed}")


def test_fused_attention_empty(ck, dev):
    e = torch.empty((0, 2, 16, 1024), dtype=torch.float16, device="cuda")
    assert tuple(ck.p97.fused_attention_cuda(e, e, e).shape) == (0, 2, 16, 1024)
