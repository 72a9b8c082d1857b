"""The attention block's stream-ordered entry point (dsv4_gpu_attn_step_d)
keeps every launch of a step on the caller's stream: on the default stream
(NULL, what torch's current stream is unless the caller picks another) and
on a created stream it gives the bits of the host-buffer entry point
(dsv4_gpu_attn_step, which test_gpu_attn_block.py pins against the
reference's attention(), dsv4_layer.c:213-336).

The block's GEMVs of q (wq_b, the indexer's wq_b) and of the output (wo_b)
once went to the library's own stream whenever the caller passed NULL. That
stream is non-blocking, so nothing ordered them against the default stream's
launches (q's norm before wq_b, wq_b before the attention, wo_b before the
caller's next read of out). Here no step is synchronised with the host, and
each output is copied on the caller's stream right behind its step, so a
launch that ran outside the stream's order would show as different bits.

One layer at the DeepSeek-V4-Flash shapes (hidden 4096, 64 heads x 512, q_lora
1024, wo_a 8 x 1024, window 128, indexer 64 x 128), ratio 4 with index_topk 4:
from position 19 on the indexer selects on the device, so every launch of the
block runs. Synthetic weights (seeded).
"""
import ctypes

import numpy as np
import pytest

import common

pytestmark = pytest.mark.gpu

LAYER = 310
N_POS = 40
# resident matrices are keyed by host pointer: their host arrays stay
# allocated for the process, so no later array can reuse an address
_KEEP = []


def _bind(D, L, rng, keep, layer=LAYER, ratio=4, n_pos=N_POS, itop=4):
    hidden, ql, H, hd, rd, win, ol, og = 4096, 1024, 64, 512, 64, 128, 1024, 8
    ih, idd = 64, 128
    coff = 2 if ratio == 4 else 1

    def fp8(rows, cols):
        W = common.fp8_codes(rng, (rows, cols))
        S = (127 + rng.integers(-8, -3, size=((rows + 127) // 128,
                                              (cols + 127) // 128))).astype(np.uint8)
        keep.extend([W, S])
        m = D.DSV4QMat(W.ctypes.data, S.ctypes.data, D.WFP8, rows, cols, 128, 128)
        assert L.dsv4_gpu_upload(ctypes.byref(m)) == 0
        return m

    def bf16(rows, cols):
        W = common.bf16_bits((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        keep.append(W)
        m = D.DSV4QMat(W.ctypes.data, None, D.WBF16, rows, cols, 0, 0)
        assert L.dsv4_gpu_upload(ctypes.byref(m)) == 0
        return m

    def vec(n, scale=0.1, add=1.0):
        v = (rng.standard_normal(n) * scale + add).astype(np.float32)
        keep.append(v)
        return v.ctypes.data

    half = rd // 2
    th = np.arange(n_pos + 8)[:, None] / (160000.0 ** (np.arange(half) * 2.0 / rd))[None, :]
    cs, sn = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
    keep += [cs, sn]
    w = D.AttnW()
    w.wq_a, w.wq_b, w.wkv = fp8(ql, hidden), fp8(H * hd, ql), fp8(hd, hidden)
    w.wo_a, w.wo_b = fp8(og * ol, H * hd // og), fp8(hidden, og * ol)
    w.comp_wkv, w.comp_wgate = bf16(coff * hd, hidden), bf16(coff * hd, hidden)
    if ratio == 4:
        w.idx_wq_b, w.idx_wproj = fp8(ih * idd, ql), bf16(ih, hidden)
    w.q_norm, w.kv_norm, w.comp_norm = vec(ql), vec(hd), vec(hd)
    w.sink, w.comp_ape = vec(H, 1.0, 0.0), vec(ratio * coff * hd, 0.5, 0.0)
    w.rope_cos, w.rope_sin = cs.ctypes.data, sn.ctypes.data
    c = D.AttnCfg(hidden=hidden, q_lora=ql, n_heads=H, head_dim=hd, rope_dim=rd, window=win,
                  ratio=ratio, idx_heads=ih if ratio == 4 else 0, idx_dim=idd, idx_topk=itop,
                  o_groups=og, o_lora=ol, max_pos=n_pos + 8, rms_eps=1e-6)
    assert L.dsv4_gpu_attn_bind(layer, ctypes.byref(c), ctypes.byref(w)) == 0
    return hidden


def _host_steps(L, layer, X):
    out = np.zeros_like(X)
    for p in range(X.shape[0]):
        assert L.dsv4_gpu_attn_step(out[p].ctypes.data, X[p].ctypes.data, layer, p) == 0
    return out


def test_attention_step_on_default_and_created_streams(gpu, dsv4):
    import torch
    L, D = gpu, dsv4
    rng = np.random.default_rng(5)
    hidden = _bind(D, L, rng, _KEEP)
    X = (rng.standard_normal((N_POS, hidden)) * 0.5).astype(np.float32)

    # the host-buffer entry point: the library's stream, synchronised per step
    want = _host_steps(L, LAYER, X)
    assert np.isfinite(want).all() and np.abs(want).max() > 0.0

    dX = torch.from_numpy(X).to("cuda:0")
    for name in ("default", "created"):
        assert L.dsv4_gpu_attn_reset(LAYER) == 0
        s = torch.cuda.current_stream() if name == "default" else torch.cuda.Stream()
        print("attn streams: %s stream, %d positions" % (name, N_POS), flush=True)
        handle = None if name == "default" else s.cuda_stream
        outs = []
        with torch.cuda.stream(s):
            d_out = torch.empty(hidden, dtype=torch.float32, device="cuda:0")
            for p in range(N_POS):
                assert L.dsv4_gpu_attn_step_d(d_out.data_ptr(), dX[p].data_ptr(), LAYER, p,
                                              handle) == 0
                outs.append(d_out.clone())
        s.synchronize()
        got = torch.stack(outs).cpu().numpy()
        bad = np.nonzero((got.view(np.uint32) != want.view(np.uint32)).any(axis=1))[0]
        assert bad.size == 0, "%s stream: positions %s differ from the host entry point" % (
            name, bad[:8].tolist())
    assert L.dsv4_gpu_attn_reset(LAYER) == 0


@pytest.mark.parametrize("ratio", [4, 128])
def test_x_projections_in_one_launch_keep_bits(gpu, dsv4, monkeypatch, ratio):
    """The block's x projections -- FP8 wq_a and wkv, BF16 compressor wkv and
    wgate and (ratio 4) the indexer's weights_proj -- run in one launch: each
    row has the bits of its own listed GEMV launch (DSV4_GPU_XPROJ=0: an FP8
    and a BF16 listed launch), so every step's output is bit-identical; the
    same with the BF16 part on its own grid (DSV4_GPU_XPROJ_CAP=0) rather
    than within the FP8 part's."""
    L, D = gpu, dsv4
    rng = np.random.default_rng(11 + ratio)
    layer = LAYER + 500 + ratio
    hidden = _bind(D, L, rng, _KEEP, layer=layer, ratio=ratio)
    X = (rng.standard_normal((N_POS, hidden)) * 0.5).astype(np.float32)
    print("attn x projections: ratio %d, one launch" % ratio, flush=True)
    one = _host_steps(L, layer, X)
    assert np.isfinite(one).all() and np.abs(one).max() > 0.0
    assert L.dsv4_gpu_attn_reset(layer) == 0
    monkeypatch.setenv("DSV4_GPU_XPROJ_CAP", "0")
    print("attn x projections: ratio %d, one launch, BF16 on its own grid" % ratio, flush=True)
    own = _host_steps(L, layer, X)
    assert L.dsv4_gpu_attn_reset(layer) == 0
    bad = np.nonzero((one.view(np.uint32) != own.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, "positions %s differ with the BF16 grid capped" % bad[:8].tolist()
    monkeypatch.delenv("DSV4_GPU_XPROJ_CAP")
    monkeypatch.setenv("DSV4_GPU_XPROJ", "0")
    print("attn x projections: ratio %d, two launches" % ratio, flush=True)
    two = _host_steps(L, layer, X)
    assert L.dsv4_gpu_attn_reset(layer) == 0
    bad = np.nonzero((one.view(np.uint32) != two.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, "positions %s differ between one and two launches" % bad[:8].tolist()


@pytest.mark.parametrize("ratio", [4, 128])
def test_q_projections_with_prep_keep_bits(gpu, dsv4, monkeypatch, ratio):
    """The block's q GEMVs (wq_b and, from position 19 on at ratio 4, the
    indexer's wq_b) norm their workgroup's copy of qr themselves while the
    prep step's ring and compressor jobs run in the same launch: every
    step's output has the bits of the separate sequence (DSV4_GPU_QPROJ=0:
    the prep launch, qr normed in place, then the listed q GEMVs), with four
    rows per step (the default) or two (DSV4_GPU_QPROJ_R=2)."""
    L, D = gpu, dsv4
    rng = np.random.default_rng(13 + ratio)
    layer = LAYER + 600 + ratio
    hidden = _bind(D, L, rng, _KEEP, layer=layer, ratio=ratio)
    X = (rng.standard_normal((N_POS, hidden)) * 0.5).astype(np.float32)
    print("attn q projections: ratio %d, one launch" % ratio, flush=True)
    one = _host_steps(L, layer, X)
    assert np.isfinite(one).all() and np.abs(one).max() > 0.0
    assert L.dsv4_gpu_attn_reset(layer) == 0
    monkeypatch.setenv("DSV4_GPU_QPROJ_R", "2")
    print("attn q projections: ratio %d, one launch, two rows per step" % ratio, flush=True)
    one2 = _host_steps(L, layer, X)
    assert L.dsv4_gpu_attn_reset(layer) == 0
    bad = np.nonzero((one.view(np.uint32) != one2.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, "positions %s differ between four and two rows" % bad[:8].tolist()
    monkeypatch.delenv("DSV4_GPU_QPROJ_R")
    monkeypatch.setenv("DSV4_GPU_QPROJ", "0")
    print("attn q projections: ratio %d, prep then the GEMVs" % ratio, flush=True)
    two = _host_steps(L, layer, X)
    assert L.dsv4_gpu_attn_reset(layer) == 0
    bad = np.nonzero((one.view(np.uint32) != two.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, "positions %s differ between one launch and two" % bad[:8].tolist()
