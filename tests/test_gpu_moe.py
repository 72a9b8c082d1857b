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


@pytest.mark.parametrize("hidden,inter,topk", [(64, 96, 3), (4096, 2048, 6),
                                               (32, 32, 1), (512, 4096, 2)])
def test_other_shapes(gpu, dsv4, hidden, inter, topk):
    run_case(dsv4, hidden, inter, topk, 16, hidden + inter, 10.0)


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
