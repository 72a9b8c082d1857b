"""The checkpoint loader (dsv4_gpu_ckpt_*): safetensors shards straight into
HBM, the matrices resident under their device addresses.

Against the same bytes read here with numpy from the same files:
- a loaded FP8 / BF16 / FP4 matrix gives the bits of the same matrix
  uploaded from host memory (dsv4_gpu_upload), through dsv4_gpu_mmq, and
  agrees with the oracle within 1e-5;
- a row-range view of a loaded matrix (attention()'s wo_a group slice)
  resolves and runs only its rows;
- a loaded routed expert runs in the fused MoE (dsv4_gpu_moe_fp4) against
  the oracle's expert_forward + k-ordered sum;
- a whole layer loads under the binder's names (dsv4_bind.c:152-243);
- tensors spread over several shards load from each;
- absent tensors, another stored format or shape, and malformed shards are
  refused.
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import common
import oracle
import tiny_checkpoint

pytestmark = pytest.mark.gpu

TOL = 1e-5
_keep = []


@pytest.fixture(autouse=True)
def fresh_backend(gpu, dsv4):
    yield
    _keep.clear()
    dsv4.lib().dsv4_gpu_shutdown()
    assert dsv4.lib().dsv4_gpu_init() == 0


def read_shards(d):
    """name -> numpy array of the stored bytes, typed as stored."""
    dt = {"F8_E4M3": np.uint8, "F8_E8M0": np.uint8, "I8": np.uint8, "U8": np.uint8,
          "BF16": np.uint16, "F32": np.float32, "I64": np.int64}
    out = {}
    for f in sorted(os.listdir(d)):
        if not f.endswith(".safetensors"):
            continue
        raw = open(os.path.join(d, f), "rb").read()
        n = struct.unpack("<Q", raw[:8])[0]
        hdr = json.loads(raw[8:8 + n])
        for name, e in hdr.items():
            if name == "__metadata__":
                continue
            a, b = e["data_offsets"]
            out[name] = np.frombuffer(raw[8 + n + a:8 + n + b], dt[e["dtype"]]).reshape(
                e["shape"])
    return out


def open_ckpt(dsv4, d):
    ck = dsv4.lib().dsv4_gpu_ckpt_open(str(d).encode())
    assert ck
    return ck


def load(dsv4, ck, base, wdt, rows, cols):
    m = dsv4.DSV4QMat()
    rc = dsv4.lib().dsv4_gpu_ckpt_load_qmat(ck, base.encode(), wdt, rows, cols, ctypes.byref(m))
    return rc, m


def host_qmat(dsv4, t, base, wdt, rows, cols):
    W = np.ascontiguousarray(t[base + ".weight"])
    S = np.ascontiguousarray(t[base + ".scale"]) if wdt != dsv4.WBF16 else None
    _keep.extend([W, S])
    blk = {dsv4.WFP8: (128, 128), dsv4.WFP4: (1, 32), dsv4.WBF16: (0, 0)}[wdt]
    return dsv4.qmat(W, S, wdt, rows, cols, *blk), W, S


def oracle_y(dsv4, wdt, x, W, S, cols):
    if wdt == dsv4.WFP8:
        return oracle.matmul_fp8(x, W, S)
    if wdt == dsv4.WFP4:
        return oracle.matmul_fp4(x, W, S, cols)
    return oracle.matmul_bf16(x, W)


def test_loaded_matrices_match_host_upload_and_oracle(gpu, dsv4, tmp_path):
    tiny_checkpoint.write(str(tmp_path))
    t = read_shards(tmp_path)
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    c = tiny_checkpoint.CFG
    d, H, hd = c["hidden"], c["n_heads"], c["head_dim"]
    cases = [("layers.1.attn.wq_a", dsv4.WFP8, c["q_lora"], d),
             ("layers.1.attn.wq_b", dsv4.WFP8, H * hd, c["q_lora"]),
             ("layers.2.attn.wo_a", dsv4.WFP8, c["o_groups"] * c["o_lora"],
              H * hd // c["o_groups"]),
             ("layers.1.ffn.gate", dsv4.WBF16, c["n_experts"], d),
             ("layers.3.attn.compressor.wkv", dsv4.WBF16, 2 * hd, d),
             ("layers.2.ffn.experts.7.w2", dsv4.WFP4, d, c["moe_inter"]),
             ("head", dsv4.WBF16, c["vocab"], d)]
    rng = np.random.default_rng(3)
    loaded = {}
    for base, wdt, rows, cols in cases:
        rc, m = load(dsv4, ck, base, wdt, rows, cols)
        assert rc == 0, base
        assert L.dsv4_gpu_has(ctypes.byref(m)) == 1
        loaded[base] = m
        x = rng.standard_normal(cols).astype(np.float32)
        y_dev = dsv4.mmq(m, x)
        hm, W, S = host_qmat(dsv4, t, base, wdt, rows, cols)
        assert L.dsv4_gpu_upload(ctypes.byref(hm)) == 0
        y_host = dsv4.mmq(hm, x)
        assert common.bits_equal(y_dev, y_host), base
        err = common.vec_rel_err(y_dev, oracle_y(dsv4, wdt, x, W, S, cols))
        print("ckpt %s: bit-equal to the host upload, worst rel %.3g" % (base, err), flush=True)
        assert err < TOL
    # wo_a's group 1, sliced as attention() slices it (dsv4_layer.c:321-334)
    wo = loaded["layers.2.attn.wo_a"]
    ol, gw = c["o_lora"], H * hd // c["o_groups"]
    view = dsv4.DSV4QMat(wo.w + ol * gw, wo.s + (ol // 128) * ((gw + 127) // 128), dsv4.WFP8,
                         ol, gw, 128, 128)
    if ol % 128 == 0:
        assert L.dsv4_gpu_has(ctypes.byref(view)) == 1
    x = rng.standard_normal(gw).astype(np.float32)
    full = dsv4.mmq(wo, x)
    if ol % 128 == 0:
        assert common.bits_equal(dsv4.mmq(view, x), full[ol:2 * ol])
    st = dsv4.CkptStats()
    assert L.dsv4_gpu_ckpt_stats_get(ck, ctypes.byref(st)) == 0
    assert st.matrices == len(cases) and st.shards == 1 and st.bytes > 33_000_000
    L.dsv4_gpu_ckpt_close(ck)


def test_loaded_expert_runs_fused(gpu, dsv4, tmp_path):
    tiny_checkpoint.write(str(tmp_path))
    t = read_shards(tmp_path)
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    c = tiny_checkpoint.CFG
    d, inter = c["hidden"], c["moe_inter"]
    ids = [9, 2, 14, 5]
    experts = []
    for e in ids:
        ew = dsv4.DSV4ExpertW()
        assert L.dsv4_gpu_ckpt_load_expert(ck, 2, e, d, inter, ctypes.byref(ew)) == 0
        assert L.dsv4_gpu_has_expert(2, e) == 1
        assert L.dsv4_gpu_has(ctypes.byref(ew.w2)) == 1
        p = "layers.2.ffn.experts.%d." % e
        experts.append({"w1": t[p + "w1.weight"], "s1": t[p + "w1.scale"],
                        "w3": t[p + "w3.weight"], "s3": t[p + "w3.scale"],
                        "w2": t[p + "w2.weight"], "s2": t[p + "w2.scale"]})
    rng = np.random.default_rng(4)
    x = rng.standard_normal(d).astype(np.float32)
    w = common.router(rng, len(ids))
    got = dsv4.moe_fp4(x, 2, np.array(ids, np.int32), w, d, inter, 10.0)
    err = common.vec_rel_err(got, oracle.moe_fp4(x, experts, w, d, inter, 10.0))
    print("ckpt experts: fused MoE worst rel %.3g" % err, flush=True)
    assert err < TOL
    # loading a registered expert again is refused
    assert L.dsv4_gpu_ckpt_load_expert(ck, 2, 9, d, inter, None) == -1
    L.dsv4_gpu_ckpt_close(ck)


def test_load_layer_under_the_binders_names(gpu, dsv4, tmp_path):
    tiny_checkpoint.write(str(tmp_path))
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    c = tiny_checkpoint.CFG
    for layer in range(c["n_layers"]):
        ratio = c["compress_ratios"][layer]
        dims = dsv4.CkptDims(hidden=c["hidden"], q_lora=c["q_lora"], n_heads=c["n_heads"],
                             head_dim=c["head_dim"], o_groups=c["o_groups"],
                             o_lora=c["o_lora"], moe_inter=c["moe_inter"],
                             n_shared=c["n_shared"], n_experts=c["n_experts"],
                             index_n_heads=c["index_n_heads"],
                             index_head_dim=c["index_head_dim"], compress_ratio=ratio,
                             has_indexer=1 if ratio == 4 else 0)
        lm = dsv4.LayerMats()
        ex = (dsv4.DSV4ExpertW * c["n_experts"])()
        assert L.dsv4_gpu_ckpt_load_layer(ck, ctypes.byref(dims), layer, ctypes.byref(lm),
                                          ex) == 0
        names = ["wq_a", "wq_b", "wkv", "wo_a", "wo_b", "shared_w1", "shared_w2",
                 "shared_w3", "gate"]
        if ratio:
            names += ["comp_wkv", "comp_wgate"]
        if ratio == 4:
            names += ["idx_wq_b", "idx_wproj", "idx_comp_wkv", "idx_comp_wgate"]
        for nm in names:
            assert L.dsv4_gpu_has(ctypes.byref(getattr(lm, nm))) == 1, (layer, nm)
        for e in range(c["n_experts"]):
            assert L.dsv4_gpu_has_expert(layer, e) == 1
            assert L.dsv4_gpu_has(ctypes.byref(ex[e].w1)) == 1
    st = dsv4.CkptStats()
    L.dsv4_gpu_ckpt_stats_get(ck, ctypes.byref(st))
    print("ckpt: %d matrices, %d experts, %d bytes in %.4f s" %
          (st.matrices, st.experts, st.bytes, st.seconds), flush=True)
    assert st.experts == c["n_layers"] * c["n_experts"]
    L.dsv4_gpu_ckpt_close(ck)


def test_load_layer_failing_partway_rolls_back(gpu, dsv4, tmp_path):
    """A layer whose last routed expert is missing from the checkpoint (the
    dims ask for one expert more than it holds): the call fails after it
    has loaded every matrix and the other experts; nothing of it stays
    resident or registered, the HBM comes back, a retry fails the same way
    (not on an expert registered already), and the layer then loads under
    its real dims."""
    tiny_checkpoint.write(str(tmp_path))
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    c = tiny_checkpoint.CFG
    layer = 1
    ratio = c["compress_ratios"][layer]

    def dims(n_experts):
        return dsv4.CkptDims(hidden=c["hidden"], q_lora=c["q_lora"], n_heads=c["n_heads"],
                             head_dim=c["head_dim"], o_groups=c["o_groups"],
                             o_lora=c["o_lora"], moe_inter=c["moe_inter"],
                             n_shared=c["n_shared"], n_experts=n_experts,
                             index_n_heads=c["index_n_heads"],
                             index_head_dim=c["index_head_dim"], compress_ratio=ratio,
                             has_indexer=1 if ratio == 4 else 0)
    free0 = L.dsv4_gpu_free_vram()
    for attempt in range(2):
        lm = dsv4.LayerMats()
        ex = (dsv4.DSV4ExpertW * (c["n_experts"] + 1))()
        d = dims(c["n_experts"] + 1)
        assert L.dsv4_gpu_ckpt_load_layer(ck, ctypes.byref(d), layer, ctypes.byref(lm), ex) == -1
        for e in range(c["n_experts"]):
            assert L.dsv4_gpu_has_expert(layer, e) == 0, (attempt, e)
        assert lm.wq_a.w is None and ex[0].w1.w is None
        print("rollback %d: free VRAM %d -> %d" % (attempt, free0, L.dsv4_gpu_free_vram()),
              flush=True)
        assert abs(L.dsv4_gpu_free_vram() - free0) < (64 << 20)
    lm = dsv4.LayerMats()
    ex = (dsv4.DSV4ExpertW * c["n_experts"])()
    d = dims(c["n_experts"])
    assert L.dsv4_gpu_ckpt_load_layer(ck, ctypes.byref(d), layer, ctypes.byref(lm), ex) == 0
    assert L.dsv4_gpu_has(ctypes.byref(lm.wo_b)) == 1
    assert all(L.dsv4_gpu_has_expert(layer, e) == 1 for e in range(c["n_experts"]))
    L.dsv4_gpu_ckpt_close(ck)


def _write_two_shards(d):
    rng = np.random.default_rng(5)
    a = tiny_checkpoint._Writer(rng)
    a.fp8("blk.a", 256, 384)
    a.bf16("blk.b.weight", 40, 64)
    a.save(os.path.join(d, "model-00001-of-00002.safetensors"))
    b = tiny_checkpoint._Writer(rng)
    b.fp8("blk.c", 130, 256)
    b.fp4("blk.d", 64, 96)
    b.save(os.path.join(d, "model-00002-of-00002.safetensors"))


def test_tensors_over_two_shards(gpu, dsv4, tmp_path):
    _write_two_shards(str(tmp_path))
    t = read_shards(tmp_path)
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    rng = np.random.default_rng(6)
    for base, wdt, rows, cols in (("blk.a", dsv4.WFP8, 256, 384), ("blk.b", dsv4.WBF16, 40, 64),
                                  ("blk.c", dsv4.WFP8, 130, 256), ("blk.d", dsv4.WFP4, 64, 96)):
        rc, m = load(dsv4, ck, base, wdt, rows, cols)
        assert rc == 0, base
        x = rng.standard_normal(cols).astype(np.float32)
        hm, W, S = host_qmat(dsv4, t, base, wdt, rows, cols)
        err = common.vec_rel_err(dsv4.mmq(m, x), oracle_y(dsv4, wdt, x, W, S, cols))
        assert err < TOL, base
    st = dsv4.CkptStats()
    L.dsv4_gpu_ckpt_stats_get(ck, ctypes.byref(st))
    assert st.shards == 2 and st.tensors == 7
    L.dsv4_gpu_ckpt_close(ck)


def test_refusals(gpu, dsv4, tmp_path):
    _write_two_shards(str(tmp_path))
    L = dsv4.lib()
    ck = open_ckpt(dsv4, tmp_path)
    assert load(dsv4, ck, "blk.none", dsv4.WFP8, 256, 384)[0] == -1      # absent
    assert load(dsv4, ck, "blk.a", dsv4.WFP8, 255, 384)[0] == -1         # another shape
    assert load(dsv4, ck, "blk.a", dsv4.WFP4, 256, 768)[0] == -1         # another format
    assert load(dsv4, ck, "blk.b", dsv4.WFP8, 40, 64)[0] == -1           # BF16 as FP8
    assert L.dsv4_gpu_ckpt_has(ck, b"blk.c.scale") == 1
    assert L.dsv4_gpu_ckpt_has(ck, b"blk.c.bias") == 0
    L.dsv4_gpu_ckpt_close(ck)
    # malformed shards: a span that disagrees with the shape, a truncated file,
    # a header that is not JSON
    bad = tmp_path / "bad"
    for kind in ("span", "truncated", "json"):
        bad.mkdir(exist_ok=True)
        for f in os.listdir(bad):
            os.remove(bad / f)
        path = bad / "x.safetensors"
        if kind == "json":
            h = b"{not json"
            path.write_bytes(struct.pack("<Q", len(h)) + h)
        else:
            hdr = {"t.weight": {"dtype": "BF16", "shape": [4, 4],
                                "data_offsets": [0, 30 if kind == "span" else 32]}}
            j = json.dumps(hdr).encode()
            body = bytes(32 if kind == "span" else 8)
            path.write_bytes(struct.pack("<Q", len(j)) + j + body)
        assert not L.dsv4_gpu_ckpt_open(str(bad).encode()), kind
    assert not L.dsv4_gpu_ckpt_open(str(tmp_path / "missing").encode())
