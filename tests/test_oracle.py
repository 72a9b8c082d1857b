"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so a plausible mistake fails it: a wrong rebias or
subnormal start, a swapped nibble, a per-element instead of per-block scale,
an in/2 stride read at full width, a missing ReLU, a wrong score scale, a
sink in the numerator or the max, a lost tie-break. The known answers are
the reference's own gates (tests/unit/test_quant.c, test_matmul.c,
test_indexer.c, test_attn.c); the closed forms and the compiled reference
(oracle/_ref, built from the reference's sources) cover the rest.
"""
import math

import numpy as np
import pytest

import common
import oracle

ref_only = pytest.mark.skipif(not oracle.ref_available(),
                              reason="compiled reference oracle/_ref not built")


def f32bits(v):
    return np.float32(v).view(np.uint32)


# ------------------------------------------------------------ formats
def test_e8m0_closed_form():
    """test_quant.c:39-58: 2^(b-127) exactly; 0 -> 2^-127 subnormal; 255 NaN."""
    d = oracle.dump_e8m0()
    for b in range(1, 255):
        assert d[b] == np.float32(math.ldexp(1.0, b - 127)), b
    assert d[0] == np.float32(math.ldexp(1.0, -127)) and d[0] != 0.0
    assert d[0].view(np.uint32) == 0x00400000
    assert np.isnan(d[255]) and not np.isinf(d[255])


def test_e4m3_closed_form():
    """Every code against sign * 2^(e-7) * (1 + m/8) (normal) or m * 2^-9
    (subnormal); FN: only 0x7F/0xFF are NaN, 0x7E = 448 (test_quant.c:60-102)."""
    d = oracle.dump_e4m3()
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 7
        if e == 15 and m == 7:
            assert np.isnan(d[b]), b
            continue
        v = s * (m * 2.0 ** -9 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8))
        assert f32bits(d[b]) == f32bits(v), (b, d[b], v)
    assert d[0x7E] == 448.0 and d[0x7B] == 352.0 and d[0x38] == 1.0
    assert d[0x01] == 2.0 ** -9 and d[0x07] == 7 * 2.0 ** -9
    assert np.nanmax(d) == 448.0
    assert f32bits(d[0x80]) == 0x80000000          # -0.0 keeps its sign


def test_e2m1_table_and_nibble_order():
    """test_quant.c:104-189: eight magnitudes, max 6, sign in bit 3;
    element 0 is the LOW nibble (0x21 -> {0.5, 1.0})."""
    d = oracle.dump_e2m1()
    mags = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    for i in range(8):
        assert d[i] == mags[i]
        assert d[i + 8] == -mags[i]
    assert f32bits(d[8]) == 0x80000000
    W = np.array([[0x21] * 16], np.uint8)               # 32 elements
    S = np.array([[127]], np.uint8)
    x = np.zeros(32, np.float32)
    x[0] = 1.0                                           # picks element 0
    assert oracle.matmul_fp4(x, W, S, 32)[0] == 0.5
    x[:] = 0
    x[1] = 1.0                                           # element 1
    assert oracle.matmul_fp4(x, W, S, 32)[0] == 1.0


# ------------------------------------------------------------ matmuls
def test_fp8_known_answers():
    """test_matmul.c:63-130."""
    W = np.zeros((2, 128), np.uint8)
    W[0], W[1] = 0x38, 0x40
    y = oracle.matmul_fp8(np.ones(128, np.float32), W, np.array([[128]], np.uint8))
    assert list(y) == [256.0, 512.0]
    W = np.full((256, 128), 0x38, np.uint8)
    y = oracle.matmul_fp8(np.ones(128, np.float32), W, np.array([[127], [129]], np.uint8))
    assert y[0] == 128 and y[127] == 128 and y[128] == 512 and y[255] == 512
    W = np.full((1, 256), 0x38, np.uint8)
    y = oracle.matmul_fp8(np.ones(256, np.float32), W, np.array([[127, 128]], np.uint8))
    assert y[0] == 384.0


def test_fp4_known_answers():
    """test_matmul.c:132-195."""
    W = np.full((2, 32), 0x22, np.uint8)
    S = np.array([[127, 128], [127, 127]], np.uint8)
    assert list(oracle.matmul_fp4(np.ones(64, np.float32), W, S, 64)) == [96.0, 64.0]
    W = np.zeros((2, 16), np.uint8)
    W[0], W[1] = 0x22, 0x44
    y = oracle.matmul_fp4(np.ones(32, np.float32), W, np.array([[127], [127]], np.uint8), 32)
    assert list(y) == [32.0, 64.0]
    W = np.full((1, 16), 0xA2, np.uint8)
    y = oracle.matmul_fp4(np.arange(1, 33, dtype=np.float32), W,
                          np.array([[128]], np.uint8), 32)
    assert y[0] == -32.0       # +1 on even (low nibble), -1 on odd, scale 2


def bf16_bits(v):
    return (np.asarray(v, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_bf16_known_answers():
    """Exact-representable cases (the bf16 rows of test_matmul.c): small
    integers and powers of two, every product and partial sum exact."""
    W = bf16_bits(np.array([[1.0] * 64, [2.0] * 64, [-0.5] * 64], np.float32))
    y = oracle.matmul_bf16(np.ones(64, np.float32), W)
    assert list(y) == [64.0, 128.0, -32.0]
    W = bf16_bits(np.arange(1, 38, dtype=np.float32)[None, :])      # ragged tail
    y = oracle.matmul_bf16(np.arange(1, 38, dtype=np.float32), W)
    assert y[0] == float(sum(i * i for i in range(1, 38)))


def test_bf16_against_double_math():
    """Independent of the tree: products widened to float64 and summed agree
    to within f32 rounding of the result."""
    rng = np.random.default_rng(6)
    W = common.bf16_matrix(rng, (70, 1000))
    x = rng.standard_normal(1000).astype(np.float32)
    Wd = (W.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = Wd @ x.astype(np.float64)
    got = oracle.matmul_bf16(x, W)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 1e-6


def test_argmax_known_answers():
    """dsv4_run.c:471-472: first maximum; ties to the lower index; -0.0 and
    +0.0 compare equal; a NaN is never picked unless it is at index 0."""
    assert oracle.argmax([1.0, 3.0, 2.0, 3.0]) == 1
    assert oracle.argmax([-0.0, 0.0, -1.0]) == 0
    assert oracle.argmax([0.0, -0.0]) == 0
    assert oracle.argmax([1.0, np.nan, 2.0, np.nan]) == 2
    assert oracle.argmax([np.nan, 5.0, 7.0]) == 0
    assert oracle.argmax([-np.inf, -np.inf]) == 0
    assert oracle.argmax([-np.inf, -1e30, np.inf, np.inf]) == 2


def test_argmax_against_numpy():
    """numpy's argmax is also the first maximum on NaN-free input."""
    rng = np.random.default_rng(13)
    for n in (1, 7, 1000, 129280):
        v = rng.standard_normal(n).astype(np.float32)
        v[rng.integers(0, n, 3)] = v.max()          # plant ties with the maximum
        assert oracle.argmax(v) == int(np.argmax(v))


def test_embed_row_known_answers_and_roundtrip():
    """BF16 widening is exact: 1.0 = 0x3F80, -2.0 = 0xC000, and the f32 bits
    carry the bf16 bits back unchanged; an f32 table row is copied."""
    t = np.array([[0x3F80, 0xC000, 0x0000, 0x8000], [0x7F80, 0x0001, 0x4049, 0xFF80]],
                 np.uint16)
    r = oracle.embed_row(t, 0)
    assert list(r[:2]) == [1.0, -2.0] and r[2] == 0.0 and np.signbit(r[3])
    rng = np.random.default_rng(14)
    tb = common.bf16_matrix(rng, (50, 300))
    for row in (0, 17, 49):
        got = oracle.embed_row(tb, row)
        assert np.array_equal((got.view(np.uint32) >> 16).astype(np.uint16), tb[row])
        assert np.array_equal(got.view(np.uint32) & 0xFFFF, np.zeros(300, np.uint32))
    tf = rng.standard_normal((5, 33)).astype(np.float32)
    assert np.array_equal(oracle.embed_row(tf, 3), tf[3])


def test_fp8_scale_formats_agree_for_powers_of_two():
    W, Sf, Se, x = common.fp8_problem(3, 300, 640)
    assert common.bits_equal(oracle.matmul_fp8(x, W, Sf), oracle.matmul_fp8(x, W, Se))


def test_fp8_against_double_math():
    """Independent of the tree: exact per-block products summed in float64
    agree to within f32 rounding of the result."""
    W, Sf, Se, x = common.fp8_problem(4, 130, 384)
    tab = oracle.dump_e4m3().astype(np.float64)
    Wd = tab[W]
    sc = np.repeat(np.repeat(Sf.astype(np.float64), 128, 0)[:130], 128, 1)[:, :384]
    want = (Wd * sc) @ x.astype(np.float64)
    got = oracle.matmul_fp8(x, W, Se)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 1e-6


@ref_only
def test_bf16_bit_equal_to_compiled_reference():
    rng = np.random.default_rng(12)
    for out, inn in [(37, 1000), (5, 16), (9, 7), (130, 7168)]:
        W = common.bf16_matrix(rng, (out, inn))
        x = rng.standard_normal(inn).astype(np.float32)
        a = oracle.matmul_bf16(x, W)
        assert common.bits_equal(a, oracle.ref_matmul_bf16(x, W))
        assert common.bits_equal(a, oracle.ref_matmul_bf16(x, W, scalar=True))


@ref_only
def test_fp8_fp4_bit_equal_to_compiled_reference():
    rng = np.random.default_rng(11)
    for out, inn in [(37, 256), (257, 1024), (64, 7168)]:
        W = common.fp8_codes(rng, (out, inn))
        S = (120 + rng.integers(0, 15, size=((out + 127) // 128, inn // 128))).astype(np.uint8)
        x = rng.standard_normal(inn, dtype=np.float32)
        a = oracle.matmul_fp8(x, W, S)
        assert common.bits_equal(a, oracle.ref_matmul_fp8(x, W, S))
        assert common.bits_equal(a, oracle.ref_matmul_fp8(x, W, S, scalar=True))
        W4 = rng.integers(0, 256, size=(out, inn // 2), dtype=np.int32).astype(np.uint8)
        S4 = (120 + rng.integers(0, 15, size=(out, inn // 32))).astype(np.uint8)
        a = oracle.matmul_fp4(x, W4, S4, inn)
        assert common.bits_equal(a, oracle.ref_matmul_fp4(x, W4, S4, inn))
        assert common.bits_equal(a, oracle.ref_matmul_fp4(x, W4, S4, inn, scalar=True))


def test_batched_equals_gemvs():
    """test_matmul.c:318-415: nt x GEMV, bit for bit."""
    rng = np.random.default_rng(5)
    W = common.fp8_codes(rng, (37, 256))
    S = (120 + rng.integers(0, 15, size=(1, 2))).astype(np.uint8)
    X = rng.standard_normal((5, 256), dtype=np.float32)
    Y = oracle.matmul_fp8(X, W, S)
    for t in range(5):
        assert common.bits_equal(Y[t], oracle.matmul_fp8(X[t], W, S))


# ------------------------------------------------------------ swiglu / moe
def test_swiglu_limits():
    g = np.array([-30, -12, -1, 0, 1, 9.5, 12, 40], np.float32)
    u = np.array([-20, 5, -11, 3, 11, -0.5, 12, -15], np.float32)
    y0 = oracle.swiglu(g, u, 0.0)
    gd = g.astype(np.float64)
    silu = gd / (1 + np.exp(-gd))
    assert np.allclose(y0, silu * u, rtol=1e-6, atol=0)
    y = oracle.swiglu(g, u, 10.0)
    gc = np.minimum(gd, 10.0)          # upper clamp only on gate
    uc = np.clip(u.astype(np.float64), -10, 10)
    assert np.allclose(y, gc / (1 + np.exp(-gc)) * uc, rtol=1e-6, atol=0)
    assert y[0] != 0.0 and abs(y[0]) < 1e-9     # gate -30 not clamped up to -10


@ref_only
def test_swiglu_bit_equal_to_compiled_reference():
    rng = np.random.default_rng(6)
    g = (rng.standard_normal(4096) * 8).astype(np.float32)
    u = (rng.standard_normal(4096) * 8).astype(np.float32)
    for lim in (10.0, 0.0, -1.0):
        assert common.bits_equal(oracle.swiglu(g, u, lim), oracle.ref_swiglu(g, u, lim))


def test_moe_is_k_ordered_expert_sum():
    rng = np.random.default_rng(7)
    hidden, inter, topk = 64, 96, 3
    ex = [common.fp4_expert(rng, hidden, inter) for _ in range(topk)]
    x = rng.standard_normal(hidden, dtype=np.float32)
    w = common.router(rng, topk)
    out, acc = oracle.moe_fp4(x, ex, w, hidden, inter, 10.0, return_acc=True)
    for k, e in enumerate(ex):
        g = oracle.matmul_fp4(x, e["w1"], e["s1"], hidden)
        u = oracle.matmul_fp4(x, e["w3"], e["s3"], hidden)
        h = oracle.swiglu(g, u, 10.0)
        assert common.bits_equal(acc[k], oracle.matmul_fp4(h, e["w2"], e["s2"], inter))
    want = np.zeros(hidden, np.float32)
    for k in range(topk):
        want = (want + (w[k] * acc[k]).astype(np.float32)).astype(np.float32)
    assert common.bits_equal(out, want)


@pytest.mark.skipif(not oracle.ref_moe_available(), reason="oracle/_ref/libdsv4moe.so not built")
@pytest.mark.parametrize("hidden,inter,n_exp,topk,limit", [
    (256, 128, 12, 4, 10.0), (512, 96, 20, 8, 10.0), (128, 64, 9, 6, 0.0),
    (7168, 2048, 10, 8, 10.0)])
def test_moe_bit_equal_to_reference_moe(hidden, inter, n_exp, topk, limit):
    """The oracle's routed-expert sum against the reference's own moe()
    (dsv4_layer.c:369-484, through oracle/moe_ref.c): hash routing picks
    the experts, the BF16 gate gives the weights as the model computes them,
    and the shared expert is zero, so moe()'s output is its k-ordered sum
    (:471-475) plus an exact +0.0. Bit for bit, including C3's shape."""
    rng = np.random.default_rng(hidden + inter + n_exp + topk)
    experts = [common.fp4_expert(rng, hidden, inter) for _ in range(n_exp)]
    ids = rng.permutation(n_exp)[:topk]
    gate = common.bf16_matrix(rng, (n_exp, hidden), 0.1)
    x = common.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    out, idx, w = oracle.ref_moe_routed(x, experts, ids, gate, limit, 1.5)
    assert np.array_equal(idx, ids)
    assert abs(float(w.astype(np.float64).sum()) - 1.5) < 1e-5
    got = oracle.moe_fp4(x, [experts[i] for i in idx], w, hidden, inter, limit)
    assert (got != 0.0).all()                 # so adding +0.0 keeps every bit
    assert common.bits_equal(got, out)


def _moe_n_batch(rng, n_exp, nt, topk, hidden, inter):
    table = {int(e): common.fp4_expert(rng, hidden, inter)
             for e in rng.choice(1000, n_exp, replace=False)}
    ids = np.array(sorted(table), np.int32)
    IDX = np.stack([rng.permutation(ids)[:topk] for _ in range(nt)]).astype(np.int32)
    W = np.stack([common.router(rng, topk) for _ in range(nt)])
    X = rng.standard_normal((nt, hidden)).astype(np.float32)
    return table, IDX, W, X


def test_moe_n_is_moe_per_token():
    """moe_n (dsv4_layer.c:714-855): every token's row is moe() of that token,
    bit for bit (the pair slots and the k-ordered sum of :829-839), and the
    distinct experts come in first-request order (:728-739)."""
    rng = np.random.default_rng(17)
    hidden, inter = 64, 96
    for n_exp, nt, topk in ((6, 7, 3), (3, 5, 3), (12, 1, 4), (9, 16, 2)):
        table, IDX, W, X = _moe_n_batch(rng, n_exp, nt, topk, hidden, inter)
        out, uniq = oracle.moe_fp4_n(X, table, IDX, W, hidden, inter, 10.0)
        want_u = []
        for e in IDX.reshape(-1):
            if int(e) not in want_u:
                want_u.append(int(e))
        assert uniq.tolist() == want_u
        for t in range(nt):
            one = oracle.moe_fp4(X[t], [table[int(e)] for e in IDX[t]], W[t], hidden, inter,
                                 10.0)
            assert common.bits_equal(out[t], one), (n_exp, nt, topk, t)


@ref_only
def test_batched_fp4_matmul_is_per_token_in_compiled_reference():
    """What makes moe_n's pair slots equal moe()'s: the compiled reference's
    dsv4_matmul_fp4_n gives every token the single-token bits of the oracle's
    (and the reference's) dsv4_matmul_fp4 -- for a gate/up and a down shape."""
    rng = np.random.default_rng(18)
    for rows, cols, nt in ((96, 64, 5), (64, 96, 9), (256, 512, 3)):
        W = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
        S = (127 + rng.integers(-6, 3, (rows, cols // 32))).astype(np.uint8)
        X = rng.standard_normal((nt, cols)).astype(np.float32)
        Y = oracle.ref_matmul_fp4_n(X, W, S, cols)
        for t in range(nt):
            assert common.bits_equal(Y[t], oracle.matmul_fp4(X[t], W, S, cols))


# ------------------------------------------------------------ indexer / top-k
def test_indexer_known_answers():
    """test_indexer.c:23-164."""
    out = oracle.indexer_score(np.array([[1, 0], [0, 0]], np.float32),
                               np.array([[1, 0], [-1, 0]], np.float32),
                               np.array([1, 1], np.float32))
    assert out[0] > 0 and out[1] == 0.0 and f32bits(out[1]) == 0
    q = np.zeros((4, 16), np.float32); q[0, 0] = 1
    kv = np.zeros((1, 16), np.float32); kv[0, 0] = 1
    w = np.array([1, 0, 0, 0], np.float32)
    want = np.float32(np.float32(1) / np.sqrt(np.float32(16))) * \
        np.float32(np.float32(1) / np.sqrt(np.float32(4)))
    assert oracle.indexer_score(q, kv, w)[0] == want
    o = oracle.indexer_score(np.array([[1, 0], [0, 1]], np.float32),
                             np.array([[1, 0], [0, 1]], np.float32),
                             np.array([1, 4], np.float32))
    assert abs(o[1] / o[0] - 4) < 1e-6
    q = np.array([[1, 2, -1, 0.5]], np.float32)
    kv = np.array([[2, 1, -0.5, 1]], np.float32)
    Hm = np.array([[1, 1, 1, 1], [1, -1, 1, -1], [1, 1, -1, -1], [1, -1, -1, 1]], np.float32) * 0.5
    a = oracle.indexer_score(q, kv, np.ones(1, np.float32))
    b = oracle.indexer_score(q @ Hm.T, kv @ Hm.T, np.ones(1, np.float32))
    assert a[0] > 0.1 and abs(a[0] - b[0]) < 1e-5


def test_topk_ties_and_clamp():
    s = np.array([1, 5, 5, 2, 0, 5], np.float32)
    assert list(oracle.topk(s, 4)) == [1, 2, 5, 3]
    assert len(oracle.topk(s, 10)) == 6
    z = np.array([0.0, -0.0, 0.0, -1.0], np.float32)     # -0 ties with +0
    assert list(oracle.topk(z, 3)) == [0, 1, 2]


def test_topk_equals_stable_sort():
    rng = np.random.default_rng(8)
    for n, k in [(1000, 100), (4096, 512), (300, 300)]:
        s = rng.integers(-20, 20, size=n).astype(np.float32) * 0.25   # many ties
        want = np.lexsort((np.arange(n), -s.astype(np.float64)))[:k]
        assert list(oracle.topk(s, k)) == list(want)


def test_indexer_plumbing():
    assert list(oracle.indexer_offset([0, 3, -1, 7, -1], 128)) == [128, 131, -1, 135, -1]
    assert [oracle.indexer_navail(p, 4) for p in (0, 3, 7, 2047)] == [0, 1, 2, 512]
    n, idx = oracle.window_idxs(5, 4)
    assert n == 4 and list(idx) == [1, 0, 3, 2]
    n, idx = oracle.window_idxs(2, 4)
    assert n == 3 and list(idx) == [2, 1, 0, -1]


@ref_only
def test_indexer_topk_bit_equal_to_compiled_reference():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    kv = rng.standard_normal((3000, 128)).astype(np.float32)
    w = rng.standard_normal(16).astype(np.float32)
    s = oracle.indexer_score(q, kv, w)
    assert common.bits_equal(s, oracle.ref_indexer_score(q, kv, w))
    assert list(oracle.topk(s, 150)) == list(oracle.ref_topk(s, 150))


# ------------------------------------------------------------ attention
def test_attention_known_answers():
    """test_attn.c:21-134."""
    kv = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], 4, 1)
    o = oracle.sparse_attn(np.zeros((2, 4), np.float32), kv,
                           np.full(2, -1000, np.float32), [0, 1, 2, 3], 1.0)
    assert np.allclose(o, 2.5, atol=1e-5)
    o = oracle.sparse_attn(np.zeros((1, 2), np.float32), np.full((1, 2), 8, np.float32),
                           np.zeros(1, np.float32), [0], 1.0)
    assert abs(o[0, 0] - 4.0) < 1e-5
    o = oracle.sparse_attn(np.zeros((2, 2), np.float32), np.full((1, 2), 8, np.float32),
                           np.array([-20, 20], np.float32), [0], 1.0)
    assert abs(o[0, 0] - 8) < 1e-3 and o[1, 0] < 1e-3
    kv = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], 2, 1)
    o = oracle.sparse_attn(np.zeros((1, 2), np.float32), kv,
                           np.full(1, -1000, np.float32), [0, -1, 2, -1], 1.0)
    assert abs(o[0, 0] - 2.0) < 1e-5


def test_attention_without_sink_is_textbook_softmax():
    rng = np.random.default_rng(10)
    h, d, n, topk = 4, 24, 50, 20
    q = rng.standard_normal((h, d)).astype(np.float32)
    kv = rng.standard_normal((n, d + 8)).astype(np.float32)
    idx = rng.integers(-1, n, size=topk).astype(np.int32)
    o = oracle.sparse_attn(q, kv, None, idx, 0.2, d_v=d + 8)
    valid = idx[idx >= 0]
    s = (q.astype(np.float64) @ kv[valid, :d].T.astype(np.float64)) * 0.2
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = p @ kv[valid].astype(np.float64)
    assert np.max(np.abs(o - want)) < 1e-5


@ref_only
def test_attention_bit_equal_to_compiled_reference():
    rng = np.random.default_rng(12)
    h, d, n, topk = 8, 64, 200, 60
    q = rng.standard_normal((h, d)).astype(np.float32)
    kv = rng.standard_normal((n, d)).astype(np.float32)
    sink = rng.standard_normal(h).astype(np.float32)
    idx = rng.integers(-1, n, size=topk).astype(np.int32)
    a = oracle.sparse_attn(q, kv, sink, idx, 0.125)
    assert common.bits_equal(a, oracle.ref_sparse_attn(q, kv, sink, idx, 0.125))


# ------------------------------------------------------- attention block
def _tables(rd=16, maxpos=64, yarn=False):
    """A RoPE table as the reference builds it (dense theta 1e4, or the
    compressed layers' 1.6e5 with YaRN); numpy double math when the compiled
    reference is absent."""
    if oracle.ref_available():
        return oracle.ref_rope_table(rd, maxpos, 65536 if yarn else 0,
                                     160000.0 if yarn else 10000.0)
    i = np.arange(rd // 2)
    f = 1.0 / (10000.0 ** (2 * i / rd))
    th = np.arange(maxpos)[:, None] * f[None, :]
    return np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)


def test_rmsnorm_closed_forms():
    """A constant vector: inv = 1/sqrt(c^2 + eps); eps on the MEAN (not the
    sum): with n = 4096 the two readings differ; the weight multiplies after
    the scale."""
    n, c, eps = 4096, 0.5, 1e-2
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    y = oracle.rmsnorm(np.full(n, c, np.float32), w, eps)
    inv = np.float32(1.0 / math.sqrt(c * c + eps))
    assert common.bits_equal(y, w * (np.float32(c) * inv))
    wrong = np.float32(1.0 / math.sqrt(c * c + eps / n))
    assert not np.allclose(y, w * (np.float32(c) * wrong), rtol=1e-4)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1024).astype(np.float32) * 3
    y = oracle.rmsnorm(x, np.ones(1024, np.float32), 1e-6)
    assert abs(np.mean(y.astype(np.float64) ** 2) - 1.0) < 1e-5


@ref_only
@pytest.mark.parametrize("n", [64, 512, 1024, 7168])
def test_rmsnorm_bit_equal_to_compiled_reference(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * 2
    w = (rng.standard_normal(n) * 0.1 + 1).astype(np.float32)
    assert common.bits_equal(oracle.rmsnorm(x, w, 1e-6), oracle.ref_rmsnorm(x, w, 1e-6))


def test_rope_closed_forms():
    """Position 0 is the identity (cos 1, sin 0); inverse undoes forward; the
    NoPE head is untouched; pairs are interleaved (v[0], v[1]), not split
    halves; each pair keeps its length."""
    cs, sn = _tables()
    rng = np.random.default_rng(4)
    v = rng.standard_normal((3, 64)).astype(np.float32)
    assert common.bits_equal(oracle.rope_apply(v, 16, cs, sn, 0), v)
    r = oracle.rope_apply(v, 16, cs, sn, 7)
    assert common.bits_equal(r[:, :48], v[:, :48])
    back = oracle.rope_apply(r, 16, cs, sn, 7, inverse=True)
    assert np.max(np.abs(back - v)) < 1e-5
    p0 = v[:, 48:].reshape(3, 8, 2)
    p1 = r[:, 48:].reshape(3, 8, 2)
    assert np.allclose(np.hypot(p0[..., 0], p0[..., 1]), np.hypot(p1[..., 0], p1[..., 1]),
                       rtol=1e-5)
    # pair 0 rotated by the angle of the table's first column
    c, s = float(cs[7, 0]), float(sn[7, 0])
    a, b = float(v[0, 48]), float(v[0, 49])
    assert abs(r[0, 48] - (a * c - b * s)) < 1e-6 and abs(r[0, 49] - (a * s + b * c)) < 1e-6


@ref_only
@pytest.mark.parametrize("yarn", [False, True])
def test_rope_bit_equal_to_compiled_reference(yarn):
    cs, sn = _tables(64, 300, yarn)
    rng = np.random.default_rng(5)
    v = rng.standard_normal((4, 512)).astype(np.float32)
    for pos in (0, 1, 37, 299):
        for inv in (False, True):
            assert common.bits_equal(oracle.rope_apply(v, 64, cs, sn, pos, inv),
                                     oracle.ref_rope_apply(v, 64, cs, sn, pos, inv))


def test_head_norm_rope():
    """Each head at unit mean square after the norm (RoPE keeps lengths), the
    NoPE part exactly q * inv, the rope part exactly the reference RoPE of
    the scaled tail."""
    cs, sn = _tables()
    rng = np.random.default_rng(6)
    q = (rng.standard_normal((4, 64)) * 5).astype(np.float32)
    out = oracle.head_norm_rope(q, 16, 1e-6, cs, sn, 9)
    ms = np.mean(out.astype(np.float64) ** 2, axis=1)
    assert np.all(np.abs(ms - 1.0) < 1e-5)
    for h in range(4):
        inv = np.float32(1.0 / math.sqrt(np.sum(q[h].astype(np.float64) ** 2) / 64 + 1e-6))
        scaled = q[h] * inv
        assert common.bits_equal(out[h, :48], scaled[:48])
        rot = (oracle.ref_rope_apply if oracle.ref_available() else oracle.rope_apply)(
            scaled, 16, cs, sn, 9)
        assert common.bits_equal(out[h], rot)


def test_compressor_closed_forms():
    """Equal scores pool to the mean; one dominant slot pools to its row;
    the window closes every `ratio` tokens; ratio 4 pools its previous
    window's first halves with the current window's second halves (the first
    window's previous slots are -inf and drop out), then slides."""
    hd, ratio = 8, 8
    C = oracle.Compressor(ratio, hd, np.zeros((ratio, hd), np.float32))
    kvs = np.arange(ratio * hd, dtype=np.float32).reshape(ratio, hd)
    for p in range(ratio - 1):
        assert C.step(kvs[p], np.zeros(hd, np.float32), p) is None
    out = C.step(kvs[ratio - 1], np.zeros(hd, np.float32), ratio - 1)
    assert np.allclose(out, kvs.mean(axis=0), rtol=1e-6)
    C = oracle.Compressor(ratio, hd, np.zeros((ratio, hd), np.float32))
    for p in range(ratio):
        sc = np.full(hd, 50.0 if p == 3 else 0.0, np.float32)
        out = C.step(kvs[p], sc, p)
    assert np.allclose(out, kvs[3], rtol=1e-6)
    # ratio 4: slot layout and the slide
    r4 = 4
    C = oracle.Compressor(r4, hd, np.zeros((r4, 2 * hd), np.float32))
    rows = np.arange(2 * r4 * 2 * hd, dtype=np.float32).reshape(2 * r4, 2 * hd)
    for p in range(r4):
        out = C.step(rows[p], np.zeros(2 * hd, np.float32), p)
    assert np.allclose(out, rows[:r4, hd:].mean(axis=0), rtol=1e-6)
    for p in range(r4, 2 * r4):
        out = C.step(rows[p], np.zeros(2 * hd, np.float32), p)
    want = np.concatenate([rows[:r4, :hd], rows[r4:, hd:]]).mean(axis=0)
    assert np.allclose(out, want, rtol=1e-6)
    assert oracle.compress_rope_pos(7, 4) == 4 and oracle.compress_rope_pos(127, 128) == 0


@ref_only
@pytest.mark.parametrize("ratio,hd", [(4, 64), (8, 64), (4, 512), (128, 512)])
def test_compressor_bit_equal_to_compiled_reference(ratio, hd):
    rng = np.random.default_rng(ratio + hd)
    width = (2 if ratio == 4 else 1) * hd
    ape = rng.standard_normal((ratio, width)).astype(np.float32) * 0.5
    A, B = oracle.Compressor(ratio, hd, ape), oracle.ref_compressor(ratio, hd, ape)
    for p in range(3 * ratio if ratio < 128 else 2 * ratio):
        kv = rng.standard_normal(width).astype(np.float32)
        sc = rng.standard_normal(width).astype(np.float32) * 3
        a, b = A.step(kv, sc, p), B.step(kv, sc, p)
        assert (a is None) == (b is None)
        if a is not None:
            assert common.bits_equal(a, b), p
        assert common.bits_equal(A.kv, B.kv) and common.bits_equal(A.sc, B.sc)
