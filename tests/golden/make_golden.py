#!/usr/bin/env python3
"""Write the golden vectors under tests/golden/ from the COMPILED REFERENCE.

Every expected output here comes from the reference's own C functions,
compiled from its sources by oracle/Makefile into oracle/_ref/libdsv4ref.so
(src/core/dsv4_matmul.c, dsv4_ops.c, dsv4_indexer.c, dsv4_attn.c). The inputs
are stored beside them, except for the C4-scale case, whose 4 MB of keys are
regenerated from a seed by tests/common.py (a digest of the regenerated
inputs is stored so that generator drift is told apart from an oracle error).

Run in the container where /root/reference exists (oracle/_ref must be
built); the tests then read the .npz files with numpy.load (no pickles).

    python tests/golden/make_golden.py            # small vectors, NaN top-k,
                                                  # batched FP8 at a matrix-core shape
    python tests/golden/make_golden.py --c4       # + C4 top-2048 (~40 s)
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import common  # noqa: E402
import oracle  # noqa: E402


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8).copy()


def small():
    out = {}
    rng = np.random.default_rng(20261201)

    # FP8 GEMV, ragged both ways, E8M0 scales 2^-7..2^7 as the reference's
    # GPU gate draws them (tests/unit/test_cuda.c:103-192).
    rows, cols = 200, 528
    W = common.fp8_codes(rng, (rows, cols))
    S = rng.integers(120, 135, size=((rows + 127) // 128, (cols + 127) // 128)).astype(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.ref_matmul_fp8(x, W, S)
    assert common.bits_equal(y, oracle.ref_matmul_fp8(x, W, S, scalar=True))
    out.update(fp8_W=W, fp8_S=S, fp8_x=x, fp8_y=y)

    # Batched FP8 (dsv4_matmul_fp8_n), nt = 5.
    xn = rng.standard_normal((5, cols)).astype(np.float32)
    out.update(fp8n_x=xn, fp8n_y=oracle.ref_matmul_fp8_n(xn, W, S))

    # FP4 GEMV: nibbles uniform, E8M0 per 1x32 in [-6, 2].
    rows4, cols4 = 96, 512
    W4 = rng.integers(0, 256, size=(rows4, cols4 // 2)).astype(np.uint8)
    S4 = (127 + rng.integers(-6, 3, size=(rows4, cols4 // 32))).astype(np.uint8)
    x4 = rng.standard_normal(cols4).astype(np.float32)
    out.update(fp4_W=W4, fp4_S=S4, fp4_x=x4, fp4_y=oracle.ref_matmul_fp4(x4, W4, S4, cols4))

    # SwiGLU at the model limit and with the clamp disabled; inputs wide
    # enough to hit both clamps.
    g = (rng.standard_normal(4096) * 8).astype(np.float32)
    u = (rng.standard_normal(4096) * 8).astype(np.float32)
    out.update(swiglu_gate=g, swiglu_up=u,
               swiglu_y10=oracle.ref_swiglu(g, u, 10.0),
               swiglu_y0=oracle.ref_swiglu(g, u, 0.0))

    # Routed MoE, 4 experts: the reference's expert_forward composition
    # (dsv4_layer.c:199-206) from its own compiled matmul and swiglu, then the
    # k-ordered sum of dsv4_layer.c:471-475 in float32, each multiply and add
    # rounded separately.
    hidden, inter, topk = 256, 128, 4
    ex = [common.fp4_expert(rng, hidden, inter) for _ in range(topk)]
    xm = common.bf16_round(rng.standard_normal(hidden).astype(np.float32))
    wm = common.router(rng, topk)
    acc = []
    for e in ex:
        gg = oracle.ref_matmul_fp4(xm, e["w1"], e["s1"], hidden)
        uu = oracle.ref_matmul_fp4(xm, e["w3"], e["s3"], hidden)
        hh = oracle.ref_swiglu(gg, uu, 10.0)
        acc.append(oracle.ref_matmul_fp4(hh, e["w2"], e["s2"], inter))
    o = np.zeros(hidden, np.float32)
    for k in range(topk):
        o = (o + (np.float32(wm[k]) * acc[k]).astype(np.float32)).astype(np.float32)
    for k, e in enumerate(ex):
        for name, v in e.items():
            out["moe_%s_%d" % (name, k)] = v
    out.update(moe_x=xm, moe_w=wm, moe_out=o, moe_acc=np.stack(acc))

    # Indexer score + top-k (dsv4_indexer.c:64-106), with ties in the scores.
    H, D, n = 8, 64, 300
    q = rng.standard_normal((H, D)).astype(np.float32)
    kv = rng.standard_normal((n, D)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    sc = oracle.ref_indexer_score(q, kv, w)
    out.update(idx_q=q, idx_kv=kv, idx_w=w, idx_scores=sc,
               idx_top=oracle.ref_topk(sc, 40))
    tie = (rng.integers(0, 23, size=5000) - 11).astype(np.float32) * np.float32(0.25)
    tie[rng.integers(0, 5000, size=50)] = -0.0
    out.update(tie_scores=tie, tie_top=oracle.ref_topk(tie, 700))

    # Sparse attention in the reference's mode (d_qk = d_v): the shape of the
    # reference's own PyTorch fixture (test_oracle.c:241-253) -- h=6, d=16,
    # 24 rows, 12 slots with 3 masked, mixed sinks -- and a wider one.
    for tag, (h, d, nrow, nsel, nmask) in (("attn_s", (6, 16, 24, 12, 3)),
                                           ("attn_w", (8, 64, 256, 100, 7))):
        qa = rng.standard_normal((h, d)).astype(np.float32)
        kva = rng.standard_normal((nrow, d)).astype(np.float32)
        sink = rng.standard_normal(h).astype(np.float32) * np.float32(2.0)
        sel = rng.permutation(nrow)[:nsel].astype(np.int32)
        sel[rng.permutation(nsel)[:nmask]] = -1
        scale = np.float32(1.0) / np.sqrt(np.float32(d))
        out.update({tag + "_q": qa, tag + "_kv": kva, tag + "_sink": sink,
                    tag + "_idx": sel, tag + "_scale": np.float32(scale),
                    tag + "_o": oracle.ref_sparse_attn(qa, kva, sink, sel, float(scale))})
    # BF16 GEMV (dsv4_matmul_bf16), ragged, drawn after every case above so
    # their inputs stay the same.
    Wb = common.bf16_matrix(rng, (75, 1000))
    xb = rng.standard_normal(1000).astype(np.float32)
    yb = oracle.ref_matmul_bf16(xb, Wb)
    assert common.bits_equal(yb, oracle.ref_matmul_bf16(xb, Wb, scalar=True))
    out.update(bf16_W=Wb, bf16_x=xb, bf16_y=yb)
    np.savez_compressed(os.path.join(HERE, "golden_small.npz"), **out)
    print("golden_small.npz: %d arrays" % len(out))


def nan_topk():
    """dsv4_topk (dsv4_indexer.c:92-106) on scores holding NaNs: the
    reference's scan takes a NaN exactly when it is the lowest index not yet
    taken. Cases cover each device path: up to 4096 scores (ranked in one
    launch), more with the k-th largest in a bin of at most 4096 elements
    (direct final pass) or of more (refined), and fewer finite scores than
    k, so that bin is the NaNs' own."""
    rng = np.random.default_rng(20261202)
    cases = []

    def case(s, k):
        cases.append((np.asarray(s, np.float32), int(k)))

    s = rng.standard_normal(300).astype(np.float32)
    s[0] = np.nan
    case(s, 40)                                           # NaN at index 0
    s = rng.standard_normal(300).astype(np.float32)
    s[[37, 150, 151, 299]] = np.nan
    case(s, 100)                                          # NaNs mid-array
    s = (rng.integers(-5, 6, 300) * 0.5).astype(np.float32)
    s[0:4] = np.nan
    s[10:20] = np.nan
    s[50:55] = np.nan
    case(s, 200)                                          # runs, with ties
    s = np.full(300, np.nan, np.float32)
    case(s, 50)                                           # all NaN
    s = (rng.integers(-40, 40, 5000) * 0.25).astype(np.float32)
    s[rng.integers(0, 5000, 60)] = -0.0
    s[0:3] = np.nan
    s[40:48] = np.nan
    s[rng.integers(0, 5000, 30)] = np.nan
    case(s, 700)                                          # radix, direct
    s = rng.standard_normal(5000).astype(np.float32)
    s[rng.permutation(5000)[:3000]] = np.nan
    case(s, 2200)                                         # finite < k, direct
    s = rng.standard_normal(9000).astype(np.float32)
    s[rng.permutation(9000)[:8000]] = np.nan
    case(s, 1200)                                         # finite < k, refined
    s = np.concatenate([np.full(4200, 1.125), rng.uniform(2.0, 4.0, 300),
                        rng.uniform(-4.0, 0.5, 500)]).astype(np.float32)
    s = s[rng.permutation(s.size)]
    s[0:5] = np.nan
    s[100:110] = np.nan
    case(s, 1000)                                         # crowded bin, refined
    out = {}
    for i, (sc, k) in enumerate(cases):
        t0 = time.time()
        out["s%d" % i] = sc
        out["k%d" % i] = np.int32(k)
        out["top%d" % i] = oracle.ref_topk(sc, k)
        print("nan top-k case %d: n %d k %d, %d NaN: %.1f s"
              % (i, sc.size, k, int(np.isnan(sc).sum()), time.time() - t0))
    np.savez_compressed(os.path.join(HERE, "golden_nan_topk.npz"), **out)
    print("golden_nan_topk.npz: %d cases" % len(cases))


def c4_inputs():
    """The C4 indexer inputs, regenerated from seed 4 (tests/common.py)."""
    rng = np.random.default_rng(4)
    codes, s, deq = common.fp8_keys(rng, 32768, 128)
    q = rng.standard_normal((16, 128)).astype(np.float32)
    w = rng.standard_normal(16).astype(np.float32)
    return codes, s, deq, q, w


def fp8n_matrix_core():
    """Batched FP8 at a shape the f32 matrix-core batched kernel takes
    (columns a multiple of 64, at least 8 tokens, two token tiles, ragged):
    the reference's dsv4_matmul_fp8_n on it."""
    rng = np.random.default_rng(20261202)
    rows, cols, nt = 192, 1024, 17
    W = common.fp8_codes(rng, (rows, cols))
    S = rng.integers(120, 135, size=((rows + 127) // 128, cols // 128)).astype(np.uint8)
    x = rng.standard_normal((nt, cols)).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "golden_fp8n_mc.npz"), W=W, S=S, x=x,
                        y=oracle.ref_matmul_fp8_n(x, W, S))
    print("golden_fp8n_mc.npz written")


def c4():
    codes, s, deq, q, w = c4_inputs()
    sc = oracle.ref_indexer_score(q, deq, w)
    t0 = time.time()
    top = oracle.ref_topk(sc, 2048)
    print("reference dsv4_topk k=2048 of 32768: %.1f s" % (time.time() - t0))
    np.savez_compressed(os.path.join(HERE, "golden_c4_topk.npz"),
                        input_digest=digest(codes, s, q, w), scores=sc, top=top)
    print("golden_c4_topk.npz written")


if __name__ == "__main__":
    if not oracle.ref_available():
        sys.exit("oracle/_ref/libdsv4ref.so is not built (make -C oracle)")
    small()
    nan_topk()
    fp8n_matrix_core()
    if "--c4" in sys.argv:
        c4()
