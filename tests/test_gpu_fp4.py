"""MXFP4 GEMV (dsv4_matmul_fp4, dsv4_matmul.c:320-345) on the MI355X: FP4
matrices made resident by dsv4_gpu_upload and run through dsv4_gpu_mmq /
dsv4_gpu_mmq_n, the reference's own dispatch (dsv4_matmul.c:525-546).

Bars: within 1e-5 vector-scaled relative of the oracle and of the compiled
reference's committed golden vector; mmq_n bit-identical to mmq per token;
exact on a known answer; -1 (CPU fallback) for shapes it does not take.
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


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def fp4_matrix(rng, rows, cols, blk_r=1, blk_c=32):
    W = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    S = rng.integers(121, 130, ((rows + blk_r - 1) // blk_r, (cols + blk_c - 1) // blk_c),
                     dtype=np.uint8)
    return W, S


def resident(dsv4, W, S, rows, cols, blk_r=1, blk_c=32):
    m = dsv4.qmat(W, S, dsv4.WFP4, rows, cols, blk_r, blk_c)
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m)) == 0
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(m)) == 1
    return m


@pytest.mark.parametrize("rows,cols,blk_r,blk_c", [
    (2048, 7168, 1, 32), (7168, 2048, 1, 32),      # C3 expert shapes
    (64, 96, 1, 32), (33, 4096, 1, 32), (100, 16384, 1, 32),
    (256, 1024, 4, 64), (130, 8192, 128, 128)])
def test_mmq_fp4_matches_oracle(gpu, dsv4, rows, cols, blk_r, blk_c):
    rng = np.random.default_rng(rows * 7 + cols)
    W, S = fp4_matrix(rng, rows, cols, blk_r, blk_c)
    x = rng.standard_normal(cols).astype(np.float32)
    m = resident(dsv4, W, S, rows, cols, blk_r, blk_c)
    got = dsv4.mmq(m, x)
    want = oracle.matmul_fp4(x, W, S, cols, blk_r, blk_c)
    err = common.vec_rel_err(got, want)
    print("fp4 mmq %dx%d blk %dx%d: worst rel %.3g" % (rows, cols, blk_r, blk_c, err),
          flush=True)
    sys.stdout.flush()
    assert err < TOL


@pytest.mark.parametrize("rows,cols,blk_r,blk_c", [
    (2048, 7168, 1, 32), (33, 4096, 1, 32), (130, 8192, 128, 128)])
def test_fp4_rows_per_workgroup_keep_bits(gpu, dsv4, monkeypatch, rows, cols, blk_r, blk_c):
    """Rows per workgroup (DSV4_GPU_FP4_RPW; 4 by default) only reshape the
    grid: a wave owns whole rows, so every setting gives the default's bits,
    including ragged last workgroups."""
    rng = np.random.default_rng(rows * 5 + cols)
    W, S = fp4_matrix(rng, rows, cols, blk_r, blk_c)
    x = rng.standard_normal(cols).astype(np.float32)
    m = resident(dsv4, W, S, rows, cols, blk_r, blk_c)
    y0 = dsv4.mmq(m, x)
    assert common.vec_rel_err(y0, oracle.matmul_fp4(x, W, S, cols, blk_r, blk_c)) < TOL
    for rpw in (1, 3, 16, 32):
        monkeypatch.setenv("DSV4_GPU_FP4_RPW", str(rpw))
        print("fp4 %dx%d rows per workgroup %d" % (rows, cols, rpw), flush=True)
        assert common.bits_equal(dsv4.mmq(m, x), y0), rpw


def test_mmq_fp4_golden(gpu, dsv4):
    """The compiled reference's dsv4_matmul_fp4 output, committed as a vector."""
    G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "golden_small.npz"))
    W, S, x, y = G["fp4_W"], G["fp4_S"], G["fp4_x"], G["fp4_y"]
    rows, cols = W.shape[0], x.size
    if cols % 32:
        pytest.skip("golden shape not a multiple of 32 columns")
    m = resident(dsv4, np.ascontiguousarray(W), np.ascontiguousarray(S), rows, cols)
    got = dsv4.mmq(m, x)
    err = common.vec_rel_err(got, y)
    print("fp4 golden %dx%d: worst rel %.3g" % (rows, cols, err), flush=True)
    assert err < TOL


@pytest.mark.parametrize("rows,cols,blk_r,blk_c,nt", [
    (512, 2048, 1, 32, 5), (2048, 7168, 1, 32, 64), (7168, 2048, 1, 32, 9),
    (64, 96, 1, 32, 3), (33, 4096, 1, 32, 2), (100, 16384, 1, 32, 5),
    (256, 1024, 4, 64, 64), (130, 8192, 128, 128, 17)])
def test_mmq_n_fp4_bit_identical_per_token(gpu, dsv4, rows, cols, blk_r, blk_c, nt):
    """The batched form (one pass over the weights for the batch, ragged token
    blocks) gives every token the single-token GEMV's bits."""
    rng = np.random.default_rng(5 + rows + nt)
    W, S = fp4_matrix(rng, rows, cols, blk_r, blk_c)
    X = rng.standard_normal((nt, cols)).astype(np.float32)
    m = resident(dsv4, W, S, rows, cols, blk_r, blk_c)
    print("fp4 mmq_n %dx%d blk %dx%d nt %d" % (rows, cols, blk_r, blk_c, nt), flush=True)
    Y = dsv4.mmq_n(m, X)
    for t in range(nt):
        assert common.bits_equal(Y[t], dsv4.mmq(m, X[t])), "token %d" % t
    err = common.vec_rel_err(Y[nt - 1], oracle.matmul_fp4(X[nt - 1], W, S, cols, blk_r, blk_c))
    assert err < TOL


def test_mmq_fp4_known_answer(gpu, dsv4):
    """Every nibble code 2 (1.0), scale byte 127 (1.0), x = 1: y = cols."""
    rows, cols = 40, 4096
    W = np.full((rows, cols // 2), 0x22, np.uint8)
    S = np.full((rows, cols // 32), 127, np.uint8)
    m = resident(dsv4, W, S, rows, cols)
    got = dsv4.mmq(m, np.ones(cols, np.float32))
    assert np.array_equal(got, np.full(rows, float(cols), np.float32))


def test_mmq_fp4_row_view(gpu, dsv4):
    """A row range inside a resident FP4 matrix runs only its own rows."""
    rng = np.random.default_rng(9)
    rows, cols = 256, 1024
    W, S = fp4_matrix(rng, rows, cols)
    resident(dsv4, W, S, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    r0, n = 64, 32
    v = dsv4.DSV4QMat(W.ctypes.data + r0 * (cols // 2), S.ctypes.data + r0 * (cols // 32),
                      dsv4.WFP4, n, cols, 1, 32)
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(v)) == 1
    got = dsv4.mmq(v, x)
    want = oracle.matmul_fp4(x, W[r0:r0 + n], S[r0:r0 + n], cols)
    assert common.vec_rel_err(got, want) < TOL


@pytest.mark.parametrize("cols,blk_c", [(48, 16), (20000, 32), (100, 32)])
def test_upload_fp4_refuses_other_shapes(gpu, dsv4, cols, blk_c):
    """Shapes the GPU path does not take stay on the CPU: upload says -1."""
    rows = 8
    W = np.zeros((rows, (cols + 1) // 2), np.uint8)
    S = np.zeros((rows, (cols + blk_c - 1) // blk_c), np.uint8)
    m = dsv4.qmat(W, S, dsv4.WFP4, rows, cols, 1, blk_c)
    assert dsv4.lib().dsv4_gpu_upload(ctypes.byref(m)) == -1
    assert dsv4.lib().dsv4_gpu_has(ctypes.byref(m)) == 0
