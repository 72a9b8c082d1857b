"""The MI355X backend against golden vectors written by the COMPILED
REFERENCE (tests/golden/make_golden.py): decoders and selection bit-exact,
GEMV / MoE / attention within 1e-5 vector-scaled relative error."""
import ctypes
import os

import numpy as np
import pytest

import common

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "golden_small.npz"))
TOL = 1e-5
_keep = []


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    _keep.clear()
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def test_fp8_gemv_golden(gpu, dsv4):
    W, S = G["fp8_W"], G["fp8_S"]
    _keep.extend([W, S])
    m = dsv4.qmat(W, S)
    assert gpu.dsv4_gpu_upload(ctypes.byref(m)) == 0
    y = dsv4.mmq(m, G["fp8_x"])
    err = common.vec_rel_err(y, G["fp8_y"])
    print("fp8 golden: worst rel %.3g" % err, flush=True)
    assert err < TOL and np.argmax(y) == np.argmax(G["fp8_y"])
    yn = dsv4.mmq_n(m, G["fp8n_x"])
    assert common.vec_rel_err(yn, G["fp8n_y"]) < TOL
    for t in range(yn.shape[0]):                 # batched == per token, bitwise
        assert common.bits_equal(yn[t], dsv4.mmq(m, G["fp8n_x"][t]))


GM = np.load(os.path.join(HERE, "golden", "golden_fp8n_mc.npz"))


@pytest.mark.parametrize("slots", ["16", "32", "64", "0"])
def test_fp8_batched_matrix_core_golden(gpu, dsv4, monkeypatch, slots):
    """The compiled reference's dsv4_matmul_fp8_n at 192x1024, 17 tokens,
    against mmq_n on the f32 matrix-core batched kernel (DSV4_GPU_MFN_L
    16 / 32 / 64: four, two or one part per row, with and without the join)
    and on the launcher's rule (0: this small launch takes the VALU kernel):
    within 1e-5, and every token bit-identical to the single-token GEMV."""
    W, S, x = GM["W"], GM["S"], GM["x"]
    _keep.extend([W, S])
    m = dsv4.qmat(W, S)
    assert gpu.dsv4_gpu_upload(ctypes.byref(m)) == 0
    monkeypatch.setenv("DSV4_GPU_MFN_L", slots)
    yn = dsv4.mmq_n(m, x)
    err = common.vec_rel_err(yn, GM["y"])
    print("fp8 batched golden (L %s): worst rel %.3g" % (slots, err), flush=True)
    assert err < TOL
    for t in range(yn.shape[0]):
        assert common.bits_equal(yn[t], dsv4.mmq(m, x[t])), t


def test_moe_golden(gpu, dsv4):
    k = G["moe_w"].size
    hidden, inter = G["moe_x"].size, G["moe_w1_0"].shape[0]
    for i in range(k):
        e = {n: G["moe_%s_%d" % (n, i)] for n in ("w1", "s1", "w3", "s3", "w2", "s2")}
        _keep.append(e)
        ew = dsv4.expert(e["w1"], e["s1"], e["w3"], e["s3"], e["w2"], e["s2"], hidden, inter)
        assert gpu.dsv4_gpu_upload_expert(5, 10 + i, ctypes.byref(ew)) == 0
    got = dsv4.moe_fp4(G["moe_x"], 5, np.arange(10, 10 + k), G["moe_w"], hidden, inter, 10.0)
    err = common.vec_rel_err(got, G["moe_out"])
    print("moe golden: worst rel %.3g" % err, flush=True)
    assert err < TOL


def test_indexer_golden_bit_exact(gpu, dsv4):
    kv = G["idx_kv"]
    keys = dsv4.KV(kv.shape[0], kv.shape[1], dsv4.KV_F32)
    try:
        keys.write(0, kv)
        sc = dsv4.indexer_score(G["idx_q"], G["idx_w"], keys, kv.shape[0])
        assert common.bits_equal(sc, G["idx_scores"])
        idx = dsv4.indexer_topk(G["idx_q"], G["idx_w"], keys, kv.shape[0], 40)
        assert np.array_equal(idx, G["idx_top"])
    finally:
        keys.free()


def test_topk_ties_golden(gpu, dsv4):
    assert np.array_equal(dsv4.topk(G["tie_scores"], 700), G["tie_top"])


GN = np.load(os.path.join(HERE, "golden", "golden_nan_topk.npz"))


@pytest.mark.parametrize("case", range(8))
def test_nan_topk_golden(gpu, dsv4, case):
    """The compiled reference's dsv4_topk on scores holding NaNs, through the
    host call and the stream-ordered one: every device path (ranked up to
    4096 scores; direct and refined final passes; fewer finite than k)."""
    import torch
    s, k = GN["s%d" % case], int(GN["k%d" % case])
    want = GN["top%d" % case]
    print("nan top-k golden %d: n %d k %d, %d NaN" % (case, s.size, k, int(np.isnan(s).sum())),
          flush=True)
    assert np.array_equal(dsv4.topk(s, k), want)
    dev = torch.device("cuda:0")
    d_s = torch.from_numpy(s).to(dev)
    d_i = torch.full((k,), 7, dtype=torch.int32, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    assert dsv4.lib().dsv4_gpu_topk_d(d_i.data_ptr(), d_s.data_ptr(), s.size, k, sp) == 0
    torch.cuda.synchronize()
    assert np.array_equal(d_i.cpu().numpy(), want)


def test_c4_topk_golden(gpu, dsv4):
    """C4: 32768 fp8 keys, top-2048 -- the reference's own selection."""
    C = np.load(os.path.join(HERE, "golden", "golden_c4_topk.npz"))
    rng = np.random.default_rng(4)
    codes, s, _ = common.fp8_keys(rng, 32768, 128)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    w = rng.standard_normal(16).astype(np.float32)
    keys = dsv4.KV(32768, 128, dsv4.KV_FP8)
    try:
        keys.write(0, codes, s)
        sc = dsv4.indexer_score(q, w, keys, 32768)
        assert common.bits_equal(sc, C["scores"])
        assert np.array_equal(dsv4.indexer_topk(q, w, keys, 32768, 2048), C["top"])
    finally:
        keys.free()


@pytest.mark.parametrize("tag", ["attn_s", "attn_w"])
def test_sparse_attn_golden(gpu, dsv4, tag):
    kv = G[tag + "_kv"]
    st = dsv4.KV(kv.shape[0], kv.shape[1], dsv4.KV_F32)
    try:
        st.write(0, kv)
        o = dsv4.sparse_attn(G[tag + "_q"], st, G[tag + "_sink"], G[tag + "_idx"],
                             float(G[tag + "_scale"]))
        err = common.vec_rel_err(o, G[tag + "_o"])
        print("%s golden: worst rel %.3g" % (tag, err), flush=True)
        assert err < TOL
    finally:
        st.free()
