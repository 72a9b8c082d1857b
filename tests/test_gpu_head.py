"""The decode loop's head on the MI355X: greedy argmax (dsv4_run.c:471-472),
the head GEMV + argmax in one call, and the embedding-row gather
(include/dsv4/dsv4.h:300-314), against the oracle's restatements.

Bars: the argmax index identical to the oracle's (ties to the lower index,
-0.0 == +0.0, NaN never picked unless at index 0); the head's token identical
to the argmax of the GPU's own logits and to the oracle's pick when the
maximum is clear; embedding rows bit-identical.
"""
import ctypes

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def dev_argmax(dsv4, v):
    import torch
    dv = torch.from_numpy(np.ascontiguousarray(v, np.float32)).to("cuda:0")
    out = torch.full((1,), -7, dtype=torch.int32, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    assert dsv4.lib().dsv4_gpu_argmax_d(out.data_ptr(), dv.data_ptr(), v.size, st) == 0
    torch.cuda.synchronize()
    return int(out.item())


@pytest.mark.parametrize("n", [1, 5, 255, 256, 257, 65536, 129280, 1 << 20])
def test_argmax_random_with_ties(gpu, dsv4, n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    v[rng.integers(0, n, 4)] = v.max()               # ties with the maximum
    assert dev_argmax(dsv4, v) == oracle.argmax(v)


@pytest.mark.parametrize("case", ["zeros", "signed_zero", "nan_inside", "nan_first",
                                  "all_nan", "neg_inf", "pos_inf_tie", "last"])
def test_argmax_edge_cases(gpu, dsv4, case):
    n = 1000
    v = np.zeros(n, np.float32)
    if case == "signed_zero":
        v[:] = -0.0
        v[10] = 0.0
    elif case == "nan_inside":
        v = np.arange(n, dtype=np.float32)
        v[n - 1] = np.nan
        v[500] = np.nan
    elif case == "nan_first":
        v = np.arange(n, dtype=np.float32)
        v[0] = np.nan
    elif case == "all_nan":
        v[:] = np.nan
    elif case == "neg_inf":
        v[:] = -np.inf
    elif case == "pos_inf_tie":
        v[300] = v[700] = np.inf
    elif case == "last":
        v[n - 1] = 1e-30
    assert dev_argmax(dsv4, v) == oracle.argmax(v)


@pytest.mark.parametrize("rows,cols", [(129280, 128), (32000, 7168), (5000, 1000)])
def test_head_argmax(gpu, dsv4, rows, cols):
    rng = np.random.default_rng(rows)
    W = common.bf16_matrix(rng, (rows, cols), 0.05)
    x = rng.standard_normal(cols).astype(np.float32)
    m = dsv4.DSV4QMat(W.ctypes.data, None, dsv4.WBF16, rows, cols, 0, 0)
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m)) == 0
    tok = dsv4.lib().dsv4_gpu_head_argmax(x.ctypes.data, ctypes.byref(m))
    logits = dsv4.mmq(m, x)
    assert tok == oracle.argmax(logits)              # the GPU's own logits
    # a clear maximum: the oracle's logits pick the same token
    hot = rows // 3
    W[hot] = common.bf16_matrix(rng, (1, cols), 0.05)[0]
    xs = np.sign(((W[hot].astype(np.uint32) << 16).view(np.float32))).astype(np.float32)
    m2 = dsv4.DSV4QMat(W.ctypes.data, None, dsv4.WBF16, rows, cols, 0, 0)
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m2)) == 0
    tok2 = dsv4.lib().dsv4_gpu_head_argmax(xs.ctypes.data, ctypes.byref(m2))
    assert tok2 == oracle.argmax(oracle.matmul_bf16(xs, W)) == hot


def test_head_argmax_not_resident(gpu, dsv4):
    W = np.zeros((8, 16), np.uint16)
    m = dsv4.DSV4QMat(W.ctypes.data, None, dsv4.WBF16, 8, 16, 0, 0)
    assert dsv4.lib().dsv4_gpu_head_argmax(np.zeros(16, np.float32).ctypes.data,
                                           ctypes.byref(m)) == -1


@pytest.mark.parametrize("fmt", ["bf16", "f32"])
def test_embed_row(gpu, dsv4, fmt):
    import torch
    rng = np.random.default_rng(3)
    vocab, hidden = 1000, 7168
    if fmt == "bf16":
        T = common.bf16_matrix(rng, (vocab, hidden))
        dt = torch.from_numpy(T.view(np.int16)).to("cuda:0")
        wdt = dsv4.WBF16
    else:
        T = rng.standard_normal((vocab, hidden)).astype(np.float32)
        dt = torch.from_numpy(T).to("cuda:0")
        wdt = dsv4.WF32
    dst = torch.empty(hidden, dtype=torch.float32, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    for row in (0, 517, vocab - 1):
        assert dsv4.lib().dsv4_gpu_embed_row_d(dst.data_ptr(), dt.data_ptr(), wdt, row,
                                               hidden, st) == 0
        torch.cuda.synchronize()
        assert common.bits_equal(dst.cpu().numpy(), oracle.embed_row(T, row))
    assert dsv4.lib().dsv4_gpu_embed_row_d(dst.data_ptr(), dt.data_ptr(), 7, 0, hidden, st) == -1
