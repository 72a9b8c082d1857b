"""Pin the CPU oracle against golden vectors written by the COMPILED
REFERENCE (tests/golden/make_golden.py; oracle/_ref built from the
reference's src/core sources). Runs on the CPU and needs neither the
reference tree nor oracle/_ref, so the pinning holds wherever the tests run.

Bit-exact throughout: the oracle restates the reference's arithmetic order.
"""
import hashlib
import os

import numpy as np
import pytest

import common
import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "golden_small.npz"))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp8_gemv_golden():
    """dsv4_matmul_fp8 (AVX2 == scalar) on a 200x528 matrix, ragged in both
    block dims, E8M0 scales 2^-7..2^7."""
    y = oracle.matmul_fp8(G["fp8_x"], G["fp8_W"], G["fp8_S"])
    assert np.array_equal(bits(y), bits(G["fp8_y"]))


def test_fp8_batched_golden():
    """dsv4_matmul_fp8_n at nt = 5."""
    y = oracle.matmul_fp8(G["fp8n_x"], G["fp8_W"], G["fp8_S"])
    assert np.array_equal(bits(y), bits(G["fp8n_y"]))


GM = np.load(os.path.join(HERE, "golden", "golden_fp8n_mc.npz"))


def test_fp8_batched_matrix_core_shape_golden():
    """dsv4_matmul_fp8_n at 192x1024, 17 tokens (a shape the batched f32
    matrix-core kernel takes): the oracle bit for bit."""
    y = oracle.matmul_fp8(GM["x"], GM["W"], GM["S"])
    assert np.array_equal(bits(y), bits(GM["y"]))


def test_bf16_gemv_golden():
    y = oracle.matmul_bf16(G["bf16_x"], G["bf16_W"])
    assert np.array_equal(bits(y), bits(G["bf16_y"]))


def test_fp4_gemv_golden():
    y = oracle.matmul_fp4(G["fp4_x"], G["fp4_W"], G["fp4_S"], G["fp4_x"].size)
    assert np.array_equal(bits(y), bits(G["fp4_y"]))


@pytest.mark.parametrize("limit,key", [(10.0, "swiglu_y10"), (0.0, "swiglu_y0")])
def test_swiglu_golden(limit, key):
    y = oracle.swiglu(G["swiglu_gate"], G["swiglu_up"], limit)
    assert np.array_equal(bits(y), bits(G[key]))


def golden_experts():
    k = G["moe_w"].size
    return [{n: G["moe_%s_%d" % (n, i)] for n in ("w1", "s1", "w3", "s3", "w2", "s2")}
            for i in range(k)]


def test_moe_golden():
    """expert_forward per k from the reference's own matmul + swiglu, then the
    k-ordered, separately rounded weighted sum (dsv4_layer.c:471-475)."""
    hidden, inter = G["moe_x"].size, G["moe_w1_0"].shape[0]
    out, acc = oracle.moe_fp4(G["moe_x"], golden_experts(), G["moe_w"], hidden, inter,
                              10.0, return_acc=True)
    assert np.array_equal(bits(acc), bits(G["moe_acc"]))
    assert np.array_equal(bits(out), bits(G["moe_out"]))


def test_indexer_score_and_topk_golden():
    sc = oracle.indexer_score(G["idx_q"], G["idx_kv"], G["idx_w"])
    assert np.array_equal(bits(sc), bits(G["idx_scores"]))
    assert np.array_equal(oracle.topk(sc, 40), G["idx_top"])


def test_topk_ties_golden():
    """Quantised scores with many ties and signed zeros, k = 700 of 5000."""
    assert np.array_equal(oracle.topk(G["tie_scores"], 700), G["tie_top"])


GN = np.load(os.path.join(HERE, "golden", "golden_nan_topk.npz"))


@pytest.mark.parametrize("case", range(8))
def test_nan_topk_golden(case):
    """dsv4_topk on scores holding NaNs (at index 0, mid-array, in runs, all
    NaN, fewer finite scores than k): the reference's scan takes a NaN
    exactly when it is the lowest untaken index."""
    s, k = GN["s%d" % case], int(GN["k%d" % case])
    assert np.array_equal(oracle.topk(s, k), GN["top%d" % case])


def test_nan_topk_matches_compiled_reference():
    """Random NaN patterns over ties, against the compiled dsv4_topk."""
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(11)
    for t in range(300):
        n = int(rng.integers(1, 200))
        s = (rng.integers(-4, 5, n) * 0.5).astype(np.float32)
        s[rng.random(n) < rng.random()] = np.nan
        k = int(rng.integers(1, n + 1))
        assert np.array_equal(oracle.topk(s, k), oracle.ref_topk(s, k)), (t, n, k)


@pytest.mark.parametrize("tag", ["attn_s", "attn_w"])
def test_sparse_attn_golden(tag):
    """dsv4_sparse_attn with masked slots and per-head sinks (the shape of the
    reference's own fixture, test_oracle.c:241-253, and a wider one)."""
    o = oracle.sparse_attn(G[tag + "_q"], G[tag + "_kv"], G[tag + "_sink"],
                           G[tag + "_idx"], float(G[tag + "_scale"]))
    assert np.array_equal(bits(o), bits(G[tag + "_o"]))


def c4_inputs():
    rng = np.random.default_rng(4)
    codes, s, deq = common.fp8_keys(rng, 32768, 128)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    w = rng.standard_normal(16).astype(np.float32)
    return codes, s, deq, q, w


def test_c4_topk_golden():
    """C4 scale: the reference's dsv4_indexer_score over 32768 fp8 keys and its
    O(k^2 n) dsv4_topk at k = 2048, against the oracle."""
    C = np.load(os.path.join(HERE, "golden", "golden_c4_topk.npz"))
    codes, s, deq, q, w = c4_inputs()
    h = hashlib.sha256()
    for a in (codes, s, q, w):
        h.update(np.ascontiguousarray(a).tobytes())
    assert np.frombuffer(h.digest(), np.uint8).tobytes() == C["input_digest"].tobytes(), \
        "the seeded C4 input generator changed; regenerate the golden vectors"
    sc = oracle.indexer_score(q, deq, w)
    assert np.array_equal(bits(sc), bits(C["scores"]))
    assert np.array_equal(oracle.topk(sc, 2048), C["top"])
