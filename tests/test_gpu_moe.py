"""Fused MXFP4 routed-expert matvec on the MI355X against the CPU oracle.

C3: 8 of 256 experts at hidden 7168 / inter 2048, x = bf16(N(0,1)) widened
to f32, router weights softmax(N(0,1)); swiglu limit 10 (the model) and 0
(the configuration's literal formula). Bar: vector-scaled relative error
< 1e-5 against the oracle's expert_forward + k-ordered sum.
"""
import sys

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-5
_keep = []


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    _keep.clear()
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def upload(dsv4, layer, eid, e, hidden, inter):
    _keep.append(e)
    ew = dsv4.expert(e["w1"], e["s1"], e["w3"], e["s3"], e["w2"], e["s2"], hidden, inter)
    import ctypes
    assert dsv4.lib().dsv4_gpu_upload_expert(layer, eid, ctypes.byref(ew)) == 0


def run_case(dsv4, hidden, inter, topk, n_experts, seed, limit):
    rng = np.random.default_rng(seed)
    ids = rng.permutation(n_experts)[:topk].astype(np.int32)
    experts = {}
    for eid in ids:
        experts[int(eid)] = common.fp4_expert(rng, hidden, inter)
        upload(dsv4, 3, int(eid), experts[int(eid)], hidden, inter)
    x = common.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    w = common.router(rng, topk)
    got = dsv4.moe_fp4(x, 3, ids, w, hidden, inter, limit)
    want = oracle.moe_fp4(x, [experts[int(i)] for i in ids], w, hidden, inter, limit)
    err = common.vec_rel_err(got, want)
    print("moe h%d i%d k%d limit %g: worst rel %.3g" % (hidden, inter, topk, limit, err),
          flush=True)
    sys.stdout.flush()
    assert err < TOL
    return got, want


@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_c3_full_shape(gpu, dsv4, limit):
    run_case(dsv4, 7168, 2048, 8, 256, 0, limit)


@pytest.mark.parametrize("form", ["0", "1", "2"])
@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_c3_full_shape_each_form(gpu, dsv4, monkeypatch, limit, form):
    """Each form: DSV4_GPU_MOE_MC=0 the VALU form; the matrix-core forms
    (bf16 MFMA, activation as three bf16 terms) =1 reading the weights in
    fragment order (shapes that are multiples of 128) and =2, the default,
    staging them through LDS (multiples of 512)."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    run_case(dsv4, 7168, 2048, 8, 256, 1, limit)


@pytest.mark.parametrize("form", ["1", "2"])
@pytest.mark.parametrize("hidden,inter,topk", [(4096, 2048, 6), (1024, 512, 16),
                                               (2048, 1024, 5), (128, 128, 1),
                                               (256, 4096, 3)])
def test_matrix_core_form_other_shapes(gpu, dsv4, monkeypatch, hidden, inter, topk, form):
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    run_case(dsv4, hidden, inter, topk, 16, hidden + inter + 1, 10.0)


def test_down_pass_forms(gpu, dsv4, monkeypatch):
    """Both down-pass shapes of the VALU form (wave per expert slot with 32 or
    16 rows per workgroup) and the row-group form give the oracle's result."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", "0")
    for env in ({"DSV4_GPU_MOE_RBW": "16"}, {"DSV4_GPU_MOE_DOWNW": "0"}):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        run_case(dsv4, 7168, 2048, 8, 256, 2, 10.0)
        for k in env:
            monkeypatch.delenv(k)


@pytest.mark.parametrize("hidden,inter,topk", [(64, 96, 3), (4096, 2048, 6),
                                               (32, 32, 1), (512, 4096, 2),
                                               (1024, 512, 16), (128, 128, 1),
                                               (384, 640, 9)])
@pytest.mark.parametrize("form", ["0", "2"])
def test_other_shapes(gpu, dsv4, monkeypatch, hidden, inter, topk, form):
    """Shapes the staged form does not take fall back to the VALU form."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    run_case(dsv4, hidden, inter, topk, 16, hidden + inter, 10.0)


@pytest.mark.parametrize("form", ["0", "1", "2"])
def test_activation_dynamic_range(gpu, dsv4, monkeypatch, form):
    """x spanning twelve decades, with an all-zero 32-block, a block of f32
    subnormals and one huge block, through every form: the matrix-core forms
    carry x as three bf16 terms (hi + mid + lo), and each of these stresses a
    different edge of that split."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    hidden, inter, topk = 1024, 512, 3
    rng = np.random.default_rng(21)
    ids = np.array([2, 0, 1], np.int32)
    experts = [common.fp4_expert(rng, hidden, inter) for _ in range(topk)]
    for i, e in zip(ids, experts):
        upload(dsv4, 4, int(i), e, hidden, inter)
    x = (rng.standard_normal(hidden) * 10.0 ** rng.uniform(-6, 6, hidden)).astype(np.float32)
    x[0:32] = 0.0
    x[32:64] = np.float32(1e-40) * rng.standard_normal(32).astype(np.float32)
    x[64:96] *= np.float32(1e20)
    w = common.router(rng, topk)
    got = dsv4.moe_fp4(x, 4, ids, w, hidden, inter, 0.0)
    want = oracle.moe_fp4(x, experts, w, hidden, inter, 0.0)
    err = common.vec_rel_err(got, want)
    print("moe dynamic range: worst rel %.3g" % err, flush=True)
    assert err < TOL


@pytest.mark.parametrize("form", ["0", "2"])
def test_repeatable_bits(gpu, dsv4, monkeypatch, form):
    """The same call twice gives the same bits (fixed reduction order)."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    hidden, inter, topk = 2048, 1024, 4
    rng = np.random.default_rng(22)
    for i in range(topk):
        upload(dsv4, 6, i, common.fp4_expert(rng, hidden, inter), hidden, inter)
    x = rng.standard_normal(hidden).astype(np.float32)
    w = common.router(rng, topk)
    a = dsv4.moe_fp4(x, 6, np.arange(topk), w, hidden, inter, 10.0)
    b = dsv4.moe_fp4(x, 6, np.arange(topk), w, hidden, inter, 10.0)
    assert common.bits_equal(a, b)


def test_exact_known_answer(gpu, dsv4):
    """All nibbles code 2 (1.0), scale 1, x = 1: gate = up = hidden, clamped
    to the limit; the expert output and the weighted sum are exact."""
    hidden, inter = 64, 32
    e = dict(w1=np.full((inter, hidden // 2), 0x22, np.uint8),
             s1=np.full((inter, hidden // 32), 127, np.uint8),
             w3=np.full((inter, hidden // 2), 0x22, np.uint8),
             s3=np.full((inter, hidden // 32), 127, np.uint8),
             w2=np.full((hidden, inter // 2), 0x22, np.uint8),
             s2=np.full((hidden, inter // 32), 120, np.uint8))     # 2^-7
    upload(dsv4, 0, 5, e, hidden, inter)
    x = np.ones(hidden, np.float32)
    got = dsv4.moe_fp4(x, 0, [5], [0.5], hidden, inter, 0.0)
    want = oracle.moe_fp4(x, [e], np.array([0.5], np.float32), hidden, inter, 0.0)
    assert common.vec_rel_err(got, want) < TOL


def test_missing_expert_is_an_error(gpu, dsv4):
    hidden, inter = 64, 32
    rng = np.random.default_rng(3)
    upload(dsv4, 1, 0, common.fp4_expert(rng, hidden, inter), hidden, inter)
    with pytest.raises(RuntimeError):
        dsv4.moe_fp4(np.ones(hidden, np.float32), 1, [0, 7], [0.5, 0.5], hidden, inter, 10.0)
    with pytest.raises(RuntimeError):                       # wrong shape for the layer
        dsv4.moe_fp4(np.ones(128, np.float32), 1, [0], [1.0], 128, inter, 10.0)


def test_device_entry_point_matches_host_path(gpu, dsv4):
    import torch
    hidden, inter, topk = 7168, 2048, 8
    rng = np.random.default_rng(9)
    ids = np.arange(topk, dtype=np.int32)
    for i in ids:
        upload(dsv4, 2, int(i), common.fp4_expert(rng, hidden, inter), hidden, inter)
    x = rng.standard_normal(hidden).astype(np.float32)
    w = common.router(rng, topk)
    host = dsv4.moe_fp4(x, 2, ids, w, hidden, inter, 10.0)
    dev = torch.device("cuda:0")
    dx, di, dw = (torch.from_numpy(a).to(dev) for a in (x, ids, w))
    do = torch.empty(hidden, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert dsv4.lib().dsv4_gpu_moe_fp4_d(do.data_ptr(), dx.data_ptr(), 2, di.data_ptr(),
                                         dw.data_ptr(), topk, hidden, inter, 10.0, st) == 0
    torch.cuda.synchronize()
    assert common.bits_equal(do.cpu().numpy(), host)


@pytest.mark.parametrize("hidden,inter,topk", [(7168, 2048, 8), (4096, 2048, 6),
                                               (1024, 512, 16), (2048, 1024, 5),
                                               (512, 4096, 3), (1024, 512, 1)])
def test_one_launch_matches_two_launches(gpu, dsv4, monkeypatch, hidden, inter, topk):
    """The staged form in one launch (DSV4_GPU_MOE_FUSE=1: pass B waits per
    expert slot on pass A's arrival counters) and in two (the default) give
    the same bits; three calls in a row with different x check that every
    call leaves the counters at zero for the next and that pass B never
    reads a stale h."""
    rng = np.random.default_rng(hidden + inter + topk)
    ids = rng.permutation(16 if topk <= 16 else topk)[:topk].astype(np.int32)
    for eid in ids:
        upload(dsv4, 7, int(eid), common.fp4_expert(rng, hidden, inter), hidden, inter)
    xs = [common.bf16_round(rng.standard_normal(hidden).astype(np.float32)) for _ in range(3)]
    w = common.router(rng, topk)
    monkeypatch.setenv("DSV4_GPU_MOE_FUSE", "0")
    two = [dsv4.moe_fp4(x, 7, ids, w, hidden, inter, 10.0) for x in xs]
    monkeypatch.setenv("DSV4_GPU_MOE_FUSE", "1")
    one = [dsv4.moe_fp4(x, 7, ids, w, hidden, inter, 10.0) for x in xs]
    print("moe one launch h%d i%d k%d" % (hidden, inter, topk), flush=True)
    for a, b in zip(one, two):
        assert common.bits_equal(a, b)


def test_one_launch_missing_expert_and_graph_replays(gpu, dsv4, monkeypatch):
    """The one-launch form on device buffers: an id outside the layer's table
    gives NaN rows (as the two-launch form does) and the next call is whole
    again; then the call captured in a HIP graph and replayed, with eager
    calls between the replays, matches the eager result every time (the
    counters return to zero inside the launch, no memset is recorded)."""
    import torch
    monkeypatch.setenv("DSV4_GPU_MOE_FUSE", "1")
    hidden, inter, topk = 7168, 2048, 8
    rng = np.random.default_rng(31)
    ids = np.arange(topk, dtype=np.int32)
    for i in ids:
        upload(dsv4, 8, int(i), common.fp4_expert(rng, hidden, inter), hidden, inter)
    x = rng.standard_normal(hidden).astype(np.float32)
    w = common.router(rng, topk)
    want = dsv4.moe_fp4(x, 8, ids, w, hidden, inter, 10.0)
    dev = torch.device("cuda:0")
    dx, dw = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    bad = torch.from_numpy(np.array([0, 1, 2, 100000, 4, 5, 6, 7], np.int32)).to(dev)
    good = torch.from_numpy(ids).to(dev)
    do = torch.empty(hidden, dtype=torch.float32, device=dev)
    L = dsv4.lib()

    def call(di, st):
        assert L.dsv4_gpu_moe_fp4_d(do.data_ptr(), dx.data_ptr(), 8, di.data_ptr(),
                                    dw.data_ptr(), topk, hidden, inter, 10.0, st) == 0
    st = torch.cuda.current_stream().cuda_stream
    call(bad, st)
    torch.cuda.synchronize()
    assert np.isnan(do.cpu().numpy()).all()
    call(good, st)
    torch.cuda.synchronize()
    assert common.bits_equal(do.cpu().numpy(), want)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        call(good, s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(good, s.cuda_stream)
    for rep in range(3):
        do.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        assert common.bits_equal(do.cpu().numpy(), want), rep
        call(good, st)
        torch.cuda.synchronize()
        assert common.bits_equal(do.cpu().numpy(), want), rep
