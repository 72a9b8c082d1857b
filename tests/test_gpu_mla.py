"""Sparse-MLA decode on the MI355X: indexer score and top-k bit-exact,
attention within 1e-5 relative (C4: 16 x 128 fp8 indexer keys over 32768
entries, top-2048 with ties to the lower index, 64 heads over a 576-d bf16
latent KV with 512-d values)."""
import sys

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
_kv = []


@pytest.fixture(autouse=True)
def free_stores(gpu, dsv4):
    yield
    for kv in _kv:
        kv.free()
    _kv.clear()


def store(dsv4, rows, fmt, scales=None):
    kv = dsv4.KV(rows.shape[0], rows.shape[1], fmt)
    kv.write(0, rows, scales)
    _kv.append(kv)
    return kv


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def c4_indexer(seed, n=32768, H=16, D=128):
    rng = np.random.default_rng(seed)
    codes, s, deq = common.fp8_keys(rng, n, D)
    q = rng.standard_normal((H, D)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    return codes, s, deq, q, w


# ------------------------------------------------------------- indexer
def test_score_and_topk_c4_bit_exact(gpu, dsv4):
    codes, s, deq, q, w = c4_indexer(0)
    keys = store(dsv4, codes, dsv4.KV_FP8, s)
    got = dsv4.indexer_score(q, w, keys, codes.shape[0])
    want = oracle.indexer_score(q, deq, w)
    nbad = int(np.sum(got.view(np.uint32) != want.view(np.uint32)))
    say("indexer C4: %d of %d scores differ in bits" % (nbad, got.size))
    assert nbad == 0
    idx = dsv4.indexer_topk(q, w, keys, codes.shape[0], 2048)
    assert np.array_equal(idx, oracle.topk(want, 2048))


def test_score_f32_keys_known_answers(gpu, dsv4):
    """test_indexer.c:23-86 on the device."""
    kv = store(dsv4, np.array([[1, 0], [-1, 0]], np.float32), dsv4.KV_F32)
    out = dsv4.indexer_score(np.array([[1, 0], [0, 0]], np.float32),
                             np.array([1, 1], np.float32), kv, 2)
    assert out[0] > 0 and out[1] == 0.0
    q = np.zeros((4, 16), np.float32); q[0, 0] = 1
    kv = store(dsv4, np.eye(1, 16, dtype=np.float32), dsv4.KV_F32)
    w = np.array([1, 0, 0, 0], np.float32)
    assert common.bits_equal(dsv4.indexer_score(q, w, kv, 1),
                             oracle.indexer_score(q, np.eye(1, 16, dtype=np.float32), w))


@pytest.mark.parametrize("H,D,n", [(64, 128, 4099), (8, 16, 20), (16, 128, 1), (3, 40, 777)])
def test_score_other_shapes_bit_exact(gpu, dsv4, H, D, n):
    rng = np.random.default_rng(H * D + n)
    kv = rng.standard_normal((n, D)).astype(np.float32)
    q = rng.standard_normal((H, D)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    keys = store(dsv4, kv, dsv4.KV_F32)
    assert common.bits_equal(dsv4.indexer_score(q, w, keys, n), oracle.indexer_score(q, kv, w))


@pytest.mark.parametrize("form", ["matrix-core", "valu"])
@pytest.mark.parametrize("fmt,H,D,n", [
    ("fp8", 16, 128, 5000), ("fp8", 64, 128, 4500), ("fp8", 20, 48, 4200), ("fp8", 3, 40, 4400),
    ("bf16", 16, 128, 4400), ("bf16", 40, 64, 4500), ("f32", 16, 128, 4300),
    ("f32", 64, 128, 5000), ("f32", 7, 36, 4700), ("f32", 8, 132, 4200)])
def test_score_forms_bit_exact(gpu, dsv4, monkeypatch, form, fmt, H, D, n):
    """Both score forms, every key format, 1-4 head tiles of the matrix-core
    form (H up to 16, 32, 64) and its element-wise key loads (FP8 rows that
    are not whole 16-byte pieces, bf16, f32), plus D = 132, past the
    matrix-core form's 128 (the VALU form then runs either way). n > 4096,
    so the f32 keys do not take the few-keys kernel."""
    if form == "valu":
        monkeypatch.setenv("DSV4_GPU_SCORE_MC", "0")
    rng = np.random.default_rng(H * D + n)
    q = rng.standard_normal((H, D)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    if fmt == "fp8":
        codes, s, deq = common.fp8_keys(rng, n, D)
        keys, want_keys = store(dsv4, codes, dsv4.KV_FP8, s), deq
    elif fmt == "bf16":
        kv = common.bf16_round(rng.standard_normal((n, D)).astype(np.float32))
        keys, want_keys = store(dsv4, common.bf16_bits(kv), dsv4.KV_BF16), kv
    else:
        kv = rng.standard_normal((n, D)).astype(np.float32)
        keys, want_keys = store(dsv4, kv, dsv4.KV_F32), kv
    say("score %s %s: H %d D %d n %d" % (form, fmt, H, D, n))
    got = dsv4.indexer_score(q, w, keys, n)
    want = oracle.indexer_score(q, want_keys, w)
    nbad = int(np.sum(got.view(np.uint32) != want.view(np.uint32)))
    assert nbad == 0, "%d of %d scores differ in bits" % (nbad, n)
    if fmt == "fp8" and H == 16:
        idx = dsv4.indexer_topk(q, w, keys, n, 512)
        assert np.array_equal(idx, oracle.topk(want, 512))


def test_score_reference_addressing(gpu, dsv4):
    """dsv4_layer.c:286-289 scores the attention cache's compressed rows
    (row width hd = 512) read at the indexer's width D = 128 from row
    `window`: key_stride D, row0 = window."""
    rng = np.random.default_rng(5)
    window, ncomp, hd, H, D = 8, 40, 512, 4, 128
    cache = rng.standard_normal((window + ncomp, hd)).astype(np.float32)
    kv = store(dsv4, cache, dsv4.KV_F32)
    q = rng.standard_normal((H, D)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    got = dsv4.indexer_score(q, w, kv, ncomp, row0=window, key_stride=D)
    want = oracle.indexer_score(q, cache[window:].ravel()[:ncomp * D], w)
    assert common.bits_equal(got, want)


def test_topk_ties_and_edges(gpu, dsv4):
    s = np.array([1, 5, 5, 2, 0, 5], np.float32)
    assert list(dsv4.topk(s, 4)) == [1, 2, 5, 3]
    assert list(dsv4.topk(s, 10)) == list(oracle.topk(s, 10))
    z = np.array([0.0, -0.0, 0.0, -1.0], np.float32)
    assert list(dsv4.topk(z, 3)) == [0, 1, 2]
    assert len(dsv4.topk(s, 0)) == 0


@pytest.mark.parametrize("n,k,levels", [(32768, 2048, 40), (5000, 4096, 7), (1025, 1, 3),
                                        (3000, 3000, 1000000), (100000, 512, 1000000),
                                        (77, 13, 5), (4096, 4096, 50), (4097, 100, 50),
                                        (512, 512, 1000000), (4096, 1, 2)])
def test_topk_random_with_ties(gpu, dsv4, n, k, levels):
    rng = np.random.default_rng(n + k)
    s = (rng.integers(-levels, levels, size=n) / 8.0).astype(np.float32)
    assert np.array_equal(dsv4.topk(s, k), oracle.topk(s, k))


@pytest.mark.parametrize("n_bin,n_above,k,grid", [
    (4096, 100, 1000, 0), (4097, 100, 1000, 0), (20000, 1000, 3000, 0),
    (20000, 1000, 3000, 1024), (9000, 0, 4096, 64), (4000, 4095, 4096, 0)])
def test_topk_crowded_bin(gpu, dsv4, n_bin, n_above, k, grid):
    """n_bin scores in one level-1 bin [1, 1.25), n_above above it, the rest
    below: up to 4096 in the bin the final pass places B's elements
    directly, past that it refines the bin first. grid > 0 rounds the bin's
    scores to multiples of 1/(4 grid), so ties cross T."""
    rng = np.random.default_rng(n_bin + n_above + k + grid)
    inb = rng.uniform(1.0, 1.25, n_bin)
    if grid:
        inb = np.minimum(np.round(inb * 4 * grid) / (4 * grid), 1.2499)
    s = np.concatenate([inb, rng.uniform(2.0, 8.0, n_above),
                        rng.uniform(-4.0, 0.5, 40000 - n_bin - n_above)]).astype(np.float32)
    s = s[rng.permutation(s.size)]
    print("top-k crowded bin: n %d, %d in B, %d above, k %d" % (s.size, n_bin, n_above, k),
          flush=True)
    assert np.array_equal(dsv4.topk(s, k), oracle.topk(s, k))


def test_topk_all_equal(gpu, dsv4):
    """Both paths: the ranked one (up to 4096 scores) and the radix select."""
    for n in (9000, 4000):
        s = np.full(n, 0.25, np.float32)
        assert np.array_equal(dsv4.topk(s, 2048), np.arange(2048))


def _nan_patterns(rng, n):
    """Scores with NaNs: at index 0, a run at the start, runs and singles
    mid-array, most scores NaN, and ties among the finite ones."""
    base = (rng.integers(-30, 30, n) * 0.25).astype(np.float32)
    out = []
    s = base.copy(); s[0] = np.nan; out.append(("index 0", s))
    s = base.copy(); s[:9] = np.nan; out.append(("run at start", s))
    s = base.copy(); s[n // 3] = np.nan; s[n // 2:n // 2 + 40] = np.nan
    s[rng.integers(0, n, 25)] = np.nan; out.append(("runs mid-array", s))
    s = base.copy(); s[1:200:3] = np.nan; s[0] = -np.inf; out.append(("interleaved", s))
    s = base.copy(); s[rng.random(n) < 0.8] = np.nan; out.append(("mostly NaN", s))
    return out


@pytest.mark.parametrize("n,k", [(4000, 100), (4000, 3500), (9000, 2048), (9000, 4096),
                                 (40000, 1000)])
def test_topk_nan_scores_bit_exact(gpu, dsv4, n, k):
    """NaN scores select as the reference's scan selects them (a NaN is
    taken exactly when it is the lowest untaken index, dsv4_indexer.c:92-106),
    through the host call and the stream-ordered one, on both paths (ranked
    up to 4096 scores, radix past that); the next clean call is unaffected."""
    import torch
    L = dsv4.lib()
    rng = np.random.default_rng(n + k)
    dev = torch.device("cuda:0")
    sp = torch.cuda.current_stream().cuda_stream
    d_i = torch.zeros(k, dtype=torch.int32, device=dev)
    clean = rng.standard_normal(n).astype(np.float32)
    for tag, scores in _nan_patterns(rng, n) + [("clean", clean)]:
        want = oracle.topk(scores, k)
        say("top-k with NaNs: n %d k %d, %s (%d NaN)" % (n, k, tag, int(np.isnan(scores).sum())))
        assert np.array_equal(dsv4.topk(scores, k), want)
        d_s = torch.from_numpy(scores).to(dev)
        d_i.fill_(7)
        assert L.dsv4_gpu_topk_d(d_i.data_ptr(), d_s.data_ptr(), n, k, sp) == 0
        torch.cuda.synchronize()
        assert np.array_equal(d_i.cpu().numpy(), want)


def test_indexer_topk_nan_weight(gpu, dsv4):
    """A NaN head weight makes a score NaN wherever that head's dot is
    positive (dsv4_indexer.c:75-80); the selection is still the reference's."""
    codes, s, deq, q, w = c4_indexer(3, n=6000)
    keys = store(dsv4, codes, dsv4.KV_FP8, s)
    w = w.copy()
    w[0] = np.nan
    sc = oracle.indexer_score(q, deq, w)
    say("indexer with a NaN weight: %d of 6000 scores NaN" % int(np.isnan(sc).sum()))
    for k in (256, 4096):
        assert np.array_equal(dsv4.indexer_topk(q, w, keys, 6000, k), oracle.topk(sc, k))
    w[0] = 1.0
    got = dsv4.indexer_topk(q, w, keys, 6000, 256)
    assert np.array_equal(got, oracle.topk(oracle.indexer_score(q, deq, w), 256))


# ----------------------------------------------------------- attention
def c4_attention(seed, n=32768, h=64, d_qk=576, d_v=512, topk=2048):
    rng = np.random.default_rng(seed)
    kv = common.bf16_round(rng.standard_normal((n, d_qk)).astype(np.float32)
                           / np.float32(np.sqrt(d_qk)))
    q = rng.standard_normal((h, d_qk)).astype(np.float32)
    idx = np.sort(rng.permutation(n)[:topk]).astype(np.int32)
    return kv, q, idx


@pytest.mark.parametrize("form", ["matrix-core", "valu"])
@pytest.mark.parametrize("with_sink", [False, True])
def test_attention_c4(gpu, dsv4, monkeypatch, with_sink, form):
    if form == "valu":
        monkeypatch.setenv("DSV4_GPU_ATTN_MC", "0")
    kv, q, idx = c4_attention(1)
    h = q.shape[0]
    sink = np.random.default_rng(2).standard_normal(h).astype(np.float32) if with_sink else None
    store_ = store(dsv4, common.bf16_bits(kv), dsv4.KV_BF16)
    scale = np.float32(1.0) / np.sqrt(np.float32(576))
    got = dsv4.sparse_attn(q, store_, sink, idx, scale, d_v=512)
    want = oracle.sparse_attn(q, kv, sink, idx, scale, d_v=512)
    err = common.vec_rel_err(got, want)
    say("attention C4 %s sink=%s: worst rel %.3g" % (form, with_sink, err))
    assert err < TOL


@pytest.mark.parametrize("h,d_qk,d_v,topk", [(16, 512, 512, 200), (128, 576, 512, 333),
                                             (32, 64, 32, 64), (64, 576, 512, 1)])
def test_attention_bf16_shapes_masked(gpu, dsv4, h, d_qk, d_v, topk):
    """bf16 KV through the matrix-core form: a partial last split, masked
    (-1) slots, repeated rows, more head tiles than waves (h = 128) and
    d_v < d_qk."""
    rng = np.random.default_rng(h + d_qk + topk)
    n = 700
    kv = common.bf16_round(rng.standard_normal((n, d_qk)).astype(np.float32) * 0.1)
    q = rng.standard_normal((h, d_qk)).astype(np.float32)
    sink = rng.standard_normal(h).astype(np.float32)
    idx = rng.integers(-1, n, size=topk).astype(np.int32)
    st = store(dsv4, common.bf16_bits(kv), dsv4.KV_BF16)
    scale = np.float32(1.0) / np.sqrt(np.float32(d_qk))
    got = dsv4.sparse_attn(q, st, sink, idx, scale, d_v=d_v)
    want = oracle.sparse_attn(q, kv, sink, idx, scale, d_v=d_v)
    err = common.vec_rel_err(got, want)
    say("attention bf16 h=%d d_qk=%d d_v=%d topk=%d: worst rel %.3g" % (h, d_qk, d_v, topk, err))
    assert err < TOL


def test_attention_reference_mode(gpu, dsv4):
    """d_qk = d_v = 512 f32 KV with a per-head sink and masked slots: the
    reference's own dsv4_sparse_attn call (dsv4_layer.c:300-301)."""
    rng = np.random.default_rng(4)
    n, h, d, topk = 300, 64, 512, 200
    kv = rng.standard_normal((n, d)).astype(np.float32) * 0.05
    q = rng.standard_normal((h, d)).astype(np.float32)
    sink = rng.standard_normal(h).astype(np.float32)
    idx = rng.integers(-1, n, size=topk).astype(np.int32)
    st = store(dsv4, kv, dsv4.KV_F32)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    got = dsv4.sparse_attn(q, st, sink, idx, scale)
    want = oracle.sparse_attn(q, kv, sink, idx, scale)
    assert common.vec_rel_err(got, want) < TOL


def test_attention_known_answers(gpu, dsv4):
    """test_attn.c:21-117 on the device."""
    kv = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], 4, 1)
    st = store(dsv4, kv, dsv4.KV_F32)
    o = dsv4.sparse_attn(np.zeros((2, 4), np.float32), st, np.full(2, -1000, np.float32),
                         [0, 1, 2, 3], 1.0)
    assert np.allclose(o, 2.5, atol=1e-5)
    st2 = store(dsv4, np.full((1, 2), 8, np.float32), dsv4.KV_F32)
    o = dsv4.sparse_attn(np.zeros((1, 2), np.float32), st2, np.zeros(1, np.float32), [0], 1.0)
    assert abs(o[0, 0] - 4.0) < 1e-5
    o = dsv4.sparse_attn(np.zeros((2, 2), np.float32), st2, np.array([-20, 20], np.float32),
                         [0], 1.0)
    assert abs(o[0, 0] - 8) < 1e-3 and o[1, 0] < 1e-3
    kv = np.repeat(np.arange(1, 5, dtype=np.float32)[:, None], 2, 1)
    st3 = store(dsv4, kv, dsv4.KV_F32)
    o = dsv4.sparse_attn(np.zeros((1, 2), np.float32), st3, np.full(1, -1000, np.float32),
                         [0, -1, 2, -1], 1.0)
    assert abs(o[0, 0] - 2.0) < 1e-5
    o = dsv4.sparse_attn(np.ones((1, 2), np.float32), st3, np.full(1, 1.0, np.float32),
                         [-1, -1], 1.0)
    assert np.all(o == 0.0)                      # attends to nothing: zero


def test_attention_rejects_out_of_range_rows(gpu, dsv4):
    st = store(dsv4, np.ones((4, 8), np.float32), dsv4.KV_F32)
    with pytest.raises(RuntimeError):
        dsv4.sparse_attn(np.ones((1, 8), np.float32), st, None, [0, 4], 1.0)


# ------------------------------------------------------ the whole step
def test_mla_decode_step_c4(gpu, dsv4):
    import torch
    codes, s, deq, qi, wi = c4_indexer(7)
    kv, q, _ = c4_attention(8)
    n, k, h = 32768, 2048, 64
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_codes, d_s, d_qi, d_wi, d_q = t(codes), t(s), t(qi), t(wi), t(q)
    d_kv = t(common.bf16_bits(kv).view(np.int16))
    d_o = torch.empty((h, 512), dtype=torch.float32, device=dev)
    d_idx = torch.empty(k, dtype=torch.int32, device=dev)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(576)))
    st = torch.cuda.current_stream().cuda_stream
    rc = dsv4.lib().dsv4_gpu_mla_decode_d(
        d_o.data_ptr(), d_idx.data_ptr(), d_qi.data_ptr(), d_wi.data_ptr(), 16, 128,
        d_codes.data_ptr(), d_s.data_ptr(), dsv4.KV_FP8, 128, n, k,
        d_q.data_ptr(), d_kv.data_ptr(), dsv4.KV_BF16, 576, n, None, h, 576, 512,
        scale, st)
    assert rc == 0
    torch.cuda.synchronize()
    want_idx = oracle.topk(oracle.indexer_score(qi, deq, wi), k)
    assert np.array_equal(d_idx.cpu().numpy(), want_idx)
    want = oracle.sparse_attn(q, kv, None, want_idx, scale, d_v=512)
    err = common.vec_rel_err(d_o.cpu().numpy(), want)
    say("mla step C4: worst rel %.3g" % err)
    assert err < TOL


def _mla_step(dsv4, codes, s, qi, wi, kv, q, n, k, sink=None, h=64, d_qk=576, d_v=512):
    import torch
    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_codes, d_s, d_qi, d_wi, d_q = t(codes), t(s), t(qi), t(wi), t(q)
    d_kv = t(common.bf16_bits(kv).view(np.int16))
    d_sink = None if sink is None else t(sink)
    d_o = torch.full((h, d_v), 3.0, dtype=torch.float32, device=dev)
    d_idx = torch.full((k,), -7, dtype=torch.int32, device=dev)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d_qk)))
    st = torch.cuda.current_stream().cuda_stream
    H, D = qi.shape
    rc = dsv4.lib().dsv4_gpu_mla_decode_d(
        d_o.data_ptr(), d_idx.data_ptr(), d_qi.data_ptr(), d_wi.data_ptr(), H, D,
        d_codes.data_ptr(), d_s.data_ptr(), dsv4.KV_FP8, D, n, k,
        d_q.data_ptr(), d_kv.data_ptr(), dsv4.KV_BF16, d_qk, n,
        None if d_sink is None else d_sink.data_ptr(), h, d_qk, d_v, scale, st)
    assert rc == 0
    torch.cuda.synchronize()
    return d_o.cpu().numpy(), d_idx.cpu().numpy(), scale


@pytest.mark.parametrize("n,k,dup,sink", [
    (32768, 2048, 0, False), (32768, 4096, 0, True), (4097, 4096, 0, False), (4097, 100, 0, False),
    (5001, 700, 0, False), (20000, 1000, 37, False), (32768, 2048, 5, True), (32769, 512, 0, False)])
def test_mla_decode_selection_cases(gpu, dsv4, n, k, dup, sink):
    """The decode step end to end: the selection equal to the oracle's top-k
    of the oracle's scores, bit for bit, and the output within 1e-5 of the
    oracle's attention over it. dup > 0 repeats key rows in blocks of dup,
    so scores tie across T; n = 5001 is not a multiple of 4, k = 700 not a
    multiple of the 64-row split, n = 4097 just past the one-launch top-k."""
    rng = np.random.default_rng(n + k + dup)
    H, D, h = 16, 128, 64
    codes, s, deq = common.fp8_keys(rng, n, D)
    if dup:
        src = (np.arange(n) // dup) * dup
        codes, s, deq = codes[src], s[src], deq[src]
    qi = rng.standard_normal((H, D)).astype(np.float32)
    wi = rng.standard_normal(H).astype(np.float32)
    kv = common.bf16_round(rng.standard_normal((n, 576)).astype(np.float32)
                           / np.float32(np.sqrt(576)))
    q = rng.standard_normal((h, 576)).astype(np.float32)
    sk = rng.standard_normal(h).astype(np.float32) if sink else None
    want_idx = oracle.topk(oracle.indexer_score(qi, deq, wi), min(k, n))
    say("mla step: n %d k %d dup %d sink %s" % (n, k, dup, sink))
    o, idx, scale = _mla_step(dsv4, codes, s, qi, wi, kv, q, n, k, sk)
    assert np.array_equal(idx[:len(want_idx)], want_idx)
    want = oracle.sparse_attn(q, kv, sk, want_idx, scale, d_v=512)
    err = common.vec_rel_err(o, want)
    say("  worst rel %.3g" % err)
    assert err < TOL


@pytest.mark.parametrize("n,k", [(9000, 512), (3000, 512)])
def test_mla_decode_nan_scores(gpu, dsv4, n, k):
    """NaN scores (a NaN head weight: every row whose dot with that head is
    positive scores NaN): the step selects the reference's rows, NaN-scored
    ones included, and attends over them within 1e-5."""
    rng = np.random.default_rng(3 + n)
    H, D, h = 16, 128, 64
    codes, s, deq = common.fp8_keys(rng, n, D)
    qi = rng.standard_normal((H, D)).astype(np.float32)
    wi = np.abs(rng.standard_normal(H)).astype(np.float32)
    wi[3] = np.nan
    kv = common.bf16_round(rng.standard_normal((n, 576)).astype(np.float32) / np.float32(24))
    q = rng.standard_normal((h, 576)).astype(np.float32)
    sc = oracle.indexer_score(qi, deq, wi)
    want_idx = oracle.topk(sc, k)
    say("mla step with NaN scores: n %d k %d, %d NaN, %d selected"
        % (n, k, int(np.isnan(sc).sum()), int(np.isnan(sc[want_idx]).sum())))
    o, idx, scale = _mla_step(dsv4, codes, s, qi, wi, kv, q, n, k)
    assert np.array_equal(idx, want_idx)
    want = oracle.sparse_attn(q, kv, None, want_idx, scale, d_v=512)
    err = common.vec_rel_err(o, want)
    say("  worst rel %.3g" % err)
    assert err < TOL
