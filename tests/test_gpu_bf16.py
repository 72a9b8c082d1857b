"""BF16 GEMV (dsv4_matmul_bf16, dsv4_matmul.c:275-291) on the MI355X: BF16
matrices made resident by dsv4_gpu_upload and run through dsv4_gpu_mmq /
dsv4_gpu_mmq_n, the reference's own dispatch (dsv4_matmul.c:525-546) -- the
router gate, the compressors, the indexer's weights_proj and the LM head.

Bars: within 1e-5 vector-scaled relative of the oracle and of the compiled
reference's committed golden vector; mmq_n bit-identical to mmq per token;
exact on a known answer; row views run their own rows; -1 (CPU fallback) for
shapes it does not take.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def resident(dsv4, W, rows, cols):
    m = dsv4.DSV4QMat(W.ctypes.data, None, dsv4.WBF16, rows, cols, 0, 0)
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m)) == 0
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(m)) == 1
    return m


@pytest.mark.parametrize("rows,cols", [(129280 // 8, 7168), (16, 128), (8, 4096),
                                       (1000, 1000), (3, 8), (77, 16384), (300, 520)])
def test_mmq_bf16_matches_oracle(gpu, dsv4, rows, cols):
    rng = np.random.default_rng(rows + cols)
    W = common.bf16_matrix(rng, (rows, cols))
    x = rng.standard_normal(cols).astype(np.float32)
    m = resident(dsv4, W, rows, cols)
    got = dsv4.mmq(m, x)
    want = oracle.matmul_bf16(x, W)
    err = common.vec_rel_err(got, want)
    print("bf16 mmq %dx%d: worst rel %.3g" % (rows, cols, err), flush=True)
    sys.stdout.flush()
    assert err < TOL


def test_mmq_bf16_golden(gpu, dsv4):
    """The compiled reference's dsv4_matmul_bf16 output, committed."""
    G = np.load(os.path.join(HERE, "golden", "golden_small.npz"))
    W, x, y = np.ascontiguousarray(G["bf16_W"]), G["bf16_x"], G["bf16_y"]
    m = resident(dsv4, W, W.shape[0], W.shape[1])
    err = common.vec_rel_err(dsv4.mmq(m, x), y)
    print("bf16 golden %dx%d: worst rel %.3g" % (W.shape[0], W.shape[1], err), flush=True)
    assert err < TOL


@pytest.mark.parametrize("rows,cols,nt", [
    (640, 2048, 4), (256, 7168, 64), (33, 16384, 3), (100, 200, 9), (5, 8, 2),
    (1000, 4096, 17), (129, 1024, 64)])
def test_mmq_n_bf16_bit_identical_per_token(gpu, dsv4, rows, cols, nt):
    """The batched form (one pass over the weights for the batch, ragged token
    blocks) gives every token the single-token GEMV's bits."""
    rng = np.random.default_rng(8 + rows + nt)
    W = common.bf16_matrix(rng, (rows, cols))
    X = rng.standard_normal((nt, cols)).astype(np.float32)
    m = resident(dsv4, W, rows, cols)
    print("bf16 mmq_n %dx%d nt %d" % (rows, cols, nt), flush=True)
    Y = dsv4.mmq_n(m, X)
    for t in range(nt):
        assert common.bits_equal(Y[t], dsv4.mmq(m, X[t])), "token %d" % t
    err = common.vec_rel_err(Y[nt - 1], oracle.matmul_bf16(X[nt - 1], W))
    assert err < TOL


def test_mmq_bf16_known_answer(gpu, dsv4):
    """Weights 1.0, 2.0 and -0.5 per row, x = 1: y = cols, 2 cols, -cols/2."""
    rows, cols = 3, 4096
    W = np.empty((rows, cols), np.uint16)
    W[0], W[1], W[2] = 0x3F80, 0x4000, 0xBF00
    got = dsv4.mmq(resident(dsv4, W, rows, cols), np.ones(cols, np.float32))
    assert list(got) == [4096.0, 8192.0, -2048.0]


def test_mmq_bf16_row_view(gpu, dsv4):
    rng = np.random.default_rng(10)
    rows, cols = 512, 768
    W = common.bf16_matrix(rng, (rows, cols))
    resident(dsv4, W, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    r0, n = 100, 37
    v = dsv4.DSV4QMat(W.ctypes.data + r0 * cols * 2, None, dsv4.WBF16, n, cols, 0, 0)
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(v)) == 1
    got = dsv4.mmq(v, x)
    assert common.vec_rel_err(got, oracle.matmul_bf16(x, W[r0:r0 + n])) < TOL


@pytest.mark.parametrize("cols", [12, 20000])
def test_upload_bf16_refuses_other_shapes(gpu, dsv4, cols):
    W = np.zeros((4, cols), np.uint16)
    m = dsv4.DSV4QMat(W.ctypes.data, None, dsv4.WBF16, 4, cols, 0, 0)
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m)) == -1
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(m)) == 0
