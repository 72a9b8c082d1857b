"""The allocation-free routed-expert entry point (dsv4_gpu_moe_fp4_noalloc_d)
against the allocating one (dsv4_gpu_moe_fp4_d) on the MI355X.

The two run the same kernels, so the bar is bit equality. Three calls in a
row share the one static scratch array: the C3 shape (8 of 16 experts,
hidden 7168, inter 2048, staged matrix-core form), then smaller inputs (hidden
1024 / inter 512, and hidden 160 / inter 96, which takes the VALU form).
Stale contents left by a larger call must not reach a smaller one. A call
that needs more scratch than the array holds is refused with -1.
"""
import ctypes
import sys

import numpy as np
import pytest

import common
import oracle

pytestmark = pytest.mark.gpu


# device buffers bound into the library, kept for the whole process
_KEEP = []


def _case(dsv4, torch, layer, hidden, inter, topk, n_experts, seed):
    L = dsv4.lib()
    rng = np.random.default_rng(seed)
    keep = []
    for eid in range(n_experts):
        e = common.fp4_expert(rng, hidden, inter)
        keep.append(e)
        ew = dsv4.expert(e["w1"], e["s1"], e["w3"], e["s3"], e["w2"], e["s2"], hidden, inter)
        assert L.dsv4_gpu_upload_expert(layer, eid, ctypes.byref(ew)) == 0
    ids = rng.permutation(n_experts)[:topk].astype(np.int32)
    x = common.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    w = common.router(rng, topk)
    dev = torch.device("cuda:0")
    d_x = torch.from_numpy(x).to(dev)
    d_i = torch.from_numpy(ids).to(dev)
    d_w = torch.from_numpy(w).to(dev)
    return dict(layer=layer, hidden=hidden, inter=inter, topk=topk, ids=ids, x=x, w=w,
                experts=[keep[i] for i in ids], d_x=d_x, d_i=d_i, d_w=d_w,
                d_a=torch.full((hidden,), float("nan"), device=dev),
                d_b=torch.full((hidden,), float("nan"), device=dev))


def _call(fn, c, out, sp):
    return fn(out.data_ptr(), c["d_x"].data_ptr(), c["layer"], c["d_i"].data_ptr(),
              c["d_w"].data_ptr(), c["topk"], c["hidden"], c["inter"], 10.0, sp)


def test_noalloc_matches_allocating_entry_point(gpu, dsv4):
    import torch
    L = dsv4.lib()
    sp = torch.cuda.current_stream().cuda_stream
    cases = [_case(dsv4, torch, 41, 7168, 2048, 8, 16, 5),
             _case(dsv4, torch, 42, 1024, 512, 4, 8, 6),
             _case(dsv4, torch, 43, 160, 96, 3, 4, 7)]
    torch.cuda.synchronize()
    # the allocation-free calls first, in a row, largest to smallest
    for c in cases:
        print("noalloc: layer %d topk %d hidden %d inter %d" %
              (c["layer"], c["topk"], c["hidden"], c["inter"]), flush=True)
        assert _call(L.dsv4_gpu_moe_fp4_noalloc_d, c, c["d_a"], sp) == 0
    torch.cuda.synchronize()
    for c in cases:
        assert _call(L.dsv4_gpu_moe_fp4_d, c, c["d_b"], sp) == 0
    torch.cuda.synchronize()
    for c in cases:
        a = c["d_a"].cpu().numpy()
        b = c["d_b"].cpu().numpy()
        assert not np.isnan(a).any()
        assert common.bits_equal(a, b), "layer %d: noalloc differs from moe_fp4_d" % c["layer"]
        want = oracle.moe_fp4(c["x"], c["experts"], c["w"], c["hidden"], c["inter"], 10.0)
        err = common.vec_rel_err(a, want)
        print("noalloc layer %d: bit-equal to moe_fp4_d, worst rel vs oracle %.3g"
              % (c["layer"], err), flush=True)
        assert err < 1e-5
    # again, smallest first: the same bits whatever ran before
    for c in reversed(cases):
        c["d_a"].fill_(float("nan"))
        assert _call(L.dsv4_gpu_moe_fp4_noalloc_d, c, c["d_a"], sp) == 0
    torch.cuda.synchronize()
    for c in cases:
        assert common.bits_equal(c["d_a"].cpu().numpy(), c["d_b"].cpu().numpy())
    sys.stdout.flush()


def test_noalloc_refuses_more_scratch_than_the_array(gpu, dsv4):
    """topk 64 at inter 8192: neither matrix-core form fits its LDS, and the
    VALU form's h needs 64 x 8192 x 4 B = 2 MiB, twice the array: refused
    before any launch (the experts are registered but never read)."""
    import torch
    L = dsv4.lib()
    hidden, inter, topk = 512, 8192, 64
    dev = torch.device("cuda:0")
    w13 = torch.zeros(inter * hidden // 2, dtype=torch.uint8, device=dev)
    s13 = torch.zeros(inter * hidden // 32, dtype=torch.uint8, device=dev)
    ew = dsv4.DSV4ExpertW(
        dsv4.DSV4QMat(w13.data_ptr(), s13.data_ptr(), dsv4.WFP4, inter, hidden, 1, 32),
        dsv4.DSV4QMat(w13.data_ptr(), s13.data_ptr(), dsv4.WFP4, inter, hidden, 1, 32),
        dsv4.DSV4QMat(w13.data_ptr(), s13.data_ptr(), dsv4.WFP4, hidden, inter, 1, 32))
    assert L.dsv4_gpu_bind_expert_d(44, 0, ctypes.byref(ew)) == 0
    x = torch.zeros(hidden, device=dev)
    idx = torch.zeros(topk, dtype=torch.int32, device=dev)
    w = torch.zeros(topk, device=dev)
    out = torch.zeros(hidden, device=dev)
    rc = L.dsv4_gpu_moe_fp4_noalloc_d(out.data_ptr(), x.data_ptr(), 44, idx.data_ptr(),
                                      w.data_ptr(), topk, hidden, inter, 10.0,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == -1
    torch.cuda.synchronize()
    # the library's expert table keeps pointing at this memory (there is no
    # unbind): it stays alive until the process ends, so no later
    # allocation can reuse it under a registered expert
    _KEEP.extend([w13, s13])
