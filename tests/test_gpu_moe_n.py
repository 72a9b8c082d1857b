"""Batched routed experts (the routed half of the reference's moe_n,
dsv4_layer.c:714-855) on the MI355X: dsv4_gpu_moe_fp4_n / _n_d.

Bars:
  - every token's output row is bit-identical to the single-token call
    (dsv4_gpu_moe_fp4) on that token -- the reference's own contract, since its
    dsv4_mmq_n is bit-identical per (row, token) to dsv4_mmq and the k-ordered
    sum is per token;
  - within 1e-5 vector-scaled relative of the oracle's moe_n restatement
    (oracle.moe_fp4_n, pinned in test_oracle.py against per-token moe() and the
    compiled reference's batched FP4 matmul).
Routing draws every token's experts from a small pool, so experts repeat
across the batch (the union the reference builds) and some get more pairs
than one 5-pair pass of the kernel takes.
"""
import ctypes

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


def _setup(dsv4, layer, hidden, inter, n_pool, seed):
    rng = np.random.default_rng(seed)
    table = {}
    for eid in rng.choice(4 * n_pool, n_pool, replace=False):
        e = common.fp4_expert(rng, hidden, inter)
        table[int(eid)] = e
        _keep.append(e)
        ew = dsv4.expert(e["w1"], e["s1"], e["w3"], e["s3"], e["w2"], e["s2"], hidden, inter)
        assert dsv4.lib().dsv4_gpu_upload_expert(layer, int(eid), ctypes.byref(ew)) == 0
    return rng, table


def _batch(rng, table, nt, topk, hidden, same=False):
    ids = np.array(sorted(table), np.int32)
    first = rng.permutation(ids)[:topk]
    IDX = np.stack([first if same else rng.permutation(ids)[:topk]
                    for _ in range(nt)]).astype(np.int32)
    W = np.stack([common.router(rng, topk) for _ in range(nt)])
    X = common.bf16_round(rng.standard_normal((nt, hidden)).astype(np.float32))
    return IDX, W, X


def _check(dsv4, layer, table, IDX, W, X, hidden, inter, limit, oracle_tokens=None):
    nt, topk = IDX.shape
    print("moe_n layer %d: nt %d topk %d hidden %d inter %d, %d distinct experts" %
          (layer, nt, topk, hidden, inter, len(np.unique(IDX))), flush=True)
    got = dsv4.moe_fp4_n(X, layer, IDX, W, hidden, inter, limit)
    for t in range(nt):
        one = dsv4.moe_fp4(X[t], layer, IDX[t], W[t], hidden, inter, limit)
        assert common.bits_equal(got[t], one), "token %d" % t
    if oracle_tokens is None:
        want, _ = oracle.moe_fp4_n(X, table, IDX, W, hidden, inter, limit)
        err = common.vec_rel_err(got.reshape(-1), want.reshape(-1))
    else:
        err = 0.0
        for t in oracle_tokens:
            want = oracle.moe_fp4(X[t], [table[int(e)] for e in IDX[t]], W[t], hidden, inter,
                                  limit)
            err = max(err, common.vec_rel_err(got[t], want))
    print("moe_n: bit-identical per token; worst rel vs oracle %.3g" % err, flush=True)
    assert err < TOL


@pytest.mark.parametrize("nt", [2, 13, 64])
def test_moe_n_c3_shape(gpu, dsv4, nt):
    """C3's expert shape (hidden 7168, inter 2048, top-8) over a pool of 24
    experts: 2 to 64 tokens, about nt / 3 pairs per expert."""
    rng, table = _setup(dsv4, 5, 7168, 2048, 24, 100 + nt)
    IDX, W, X = _batch(rng, table, nt, 8, 7168)
    _check(dsv4, 5, table, IDX, W, X, 7168, 2048, 10.0,
           oracle_tokens=None if nt <= 2 else [0, nt - 1])


def test_moe_n_one_expert_set_for_every_token(gpu, dsv4):
    """64 tokens that all ask for the same 8 experts: 64 pairs per expert, so
    each expert runs 13 passes of 5 pairs over its (once-streamed) weights."""
    rng, table = _setup(dsv4, 6, 7168, 2048, 8, 7)
    IDX, W, X = _batch(rng, table, 64, 8, 7168, same=True)
    _check(dsv4, 6, table, IDX, W, X, 7168, 2048, 10.0, oracle_tokens=[0, 33, 63])


@pytest.mark.parametrize("hidden,inter,topk,nt,limit", [
    (1024, 512, 4, 9, 10.0), (4096, 1024, 6, 5, 0.0), (512, 2048, 3, 17, 10.0),
    (2048, 4096, 2, 3, 10.0), (1024, 512, 1, 64, 10.0)])
def test_moe_n_other_shapes(gpu, dsv4, hidden, inter, topk, nt, limit):
    """Unit counts other than C3's (14 / 4) take the run-time unit loop."""
    rng, table = _setup(dsv4, 7, hidden, inter, 10, hidden + inter + nt)
    IDX, W, X = _batch(rng, table, nt, topk, hidden)
    _check(dsv4, 7, table, IDX, W, X, hidden, inter, limit)


@pytest.mark.parametrize("mode", ["auto", "0", "1"])
def test_moe_n_tokenwise_rule(gpu, dsv4, monkeypatch, mode):
    """Pairs that barely share experts (4 tokens x top-8 drawn from 64
    experts): the host-buffer call then runs the tokens one by one through
    the single-token kernels (auto, or DSV4_GPU_MOEN_TOKENWISE=1); =0 keeps
    the batched kernels. Every mode gives each token its single-token bits."""
    if mode != "auto":
        monkeypatch.setenv("DSV4_GPU_MOEN_TOKENWISE", mode)
    rng, table = _setup(dsv4, 11, 2048, 1024, 64, 13)
    IDX, W, X = _batch(rng, table, 4, 8, 2048)
    _check(dsv4, 11, table, IDX, W, X, 2048, 1024, 10.0)


@pytest.mark.parametrize("form", ["0", "1"])
def test_moe_n_other_forms_go_token_by_token(gpu, dsv4, monkeypatch, form):
    """The VALU and fragment-order forms have no batched kernel: the batched
    call runs them token by token, so the bits are theirs."""
    monkeypatch.setenv("DSV4_GPU_MOE_MC", form)
    rng, table = _setup(dsv4, 8, 1024, 512, 6, 3)
    IDX, W, X = _batch(rng, table, 7, 4, 1024)
    _check(dsv4, 8, table, IDX, W, X, 1024, 512, 10.0)


def test_moe_n_device_form_and_a_missing_expert(gpu, dsv4):
    """dsv4_gpu_moe_fp4_n_d on device buffers: the rows of tokens whose
    experts are all resident match the host-buffer call bit for bit; a token
    routed to an id outside the table or not registered gets NaN, as the
    single-token device call gives it."""
    import torch
    hidden, inter, topk, nt = 1024, 512, 4, 6
    rng, table = _setup(dsv4, 9, hidden, inter, 8, 11)
    IDX, W, X = _batch(rng, table, nt, topk, hidden)
    want = dsv4.moe_fp4_n(X, 9, IDX, W, hidden, inter, 10.0)
    bad = IDX.copy()
    bad[2, 1] = 100000                       # outside the layer's table
    missing = min(set(range(max(table))) - set(table))   # inside the table, never registered
    bad[4, 3] = missing
    dev = torch.device("cuda:0")
    d_x = torch.from_numpy(X).to(dev)
    d_i = torch.from_numpy(bad).to(dev)
    d_w = torch.from_numpy(W).to(dev)
    d_o = torch.full((nt, hidden), 7.0, device=dev)
    sp = torch.cuda.current_stream().cuda_stream
    assert dsv4.lib().dsv4_gpu_moe_fp4_n_d(d_o.data_ptr(), d_x.data_ptr(), 9, d_i.data_ptr(),
                                           d_w.data_ptr(), nt, topk, hidden, inter, 10.0,
                                           sp) == 0
    torch.cuda.synchronize()
    got = d_o.cpu().numpy()
    for t in range(nt):
        if t in (2, 4):
            assert np.isnan(got[t]).all(), "token %d" % t
        else:
            assert common.bits_equal(got[t], want[t]), "token %d" % t


def test_moe_n_refusals(gpu, dsv4):
    """The host-buffer call refuses an expert that is not resident and a batch
    above DSV4_MAX_BATCH, before launching anything."""
    hidden, inter, topk = 1024, 512, 2
    rng, table = _setup(dsv4, 10, hidden, inter, 4, 12)
    IDX, W, X = _batch(rng, table, 3, topk, hidden)
    IDX[1, 0] = max(table) + 1
    with pytest.raises(RuntimeError):
        dsv4.moe_fp4_n(X, 10, IDX, W, hidden, inter, 10.0)
    IDX, W, X = _batch(rng, table, 65, topk, hidden)
    with pytest.raises(RuntimeError):
        dsv4.moe_fp4_n(X, 10, IDX, W, hidden, inter, 10.0)
