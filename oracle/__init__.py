"""CPU checker for the decode hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the thing results
are checked against (or timed beside). The shipped library never links,
calls or falls back to it.

Two CPU implementations are exposed through ctypes:

* ``liboracle.so`` -- this directory's C restatement (``dsv4_oracle.c``) of
  the reference functions, each citing the reference file:line it follows.
* ``_ref/libdsv4ref.so`` -- the reference's own sources
  (``src/core/dsv4_{matmul,indexer,attn,ops,rope,compress}.c``) compiled as they lie by
  ``oracle/Makefile``. Present wherever it was built; used to pin the
  restatement bit for bit and as the ``cpu_baseline`` of ``bench.py``.
* ``_ref/libdsv4moe.so`` -- the reference's static ``moe()``
  (``src/model/dsv4_layer.c:369-484``) reached through ``moe_ref.c``, which
  #includes that file; pins the restatement's routed-expert sum.

Parity unpinned: none of the restatement's functions. Each is checked
against the compiled reference in its reference-shaped special case and
against closed forms / known answers for the generalisations (see tests/).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_ORC_PATH = os.path.join(HERE, "liboracle.so")
_REF_PATH = os.path.join(HERE, "_ref", "libdsv4ref.so")
_MOE_PATH = os.path.join(HERE, "_ref", "libdsv4moe.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_vp = ctypes.c_void_p

_orc = None
_ref = None
_moe = None


def build():
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def lib():
    global _orc
    if _orc is None:
        if not os.path.exists(_ORC_PATH):
            build()
        L = ctypes.CDLL(_ORC_PATH)
        L.orc_e4m3_to_f32.restype = ctypes.c_float
        L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_to_f32.restype = ctypes.c_float
        L.orc_e8m0_to_f32.argtypes = [ctypes.c_uint8]
        L.orc_e2m1_to_f32.restype = ctypes.c_float
        L.orc_e2m1_to_f32.argtypes = [ctypes.c_uint8]
        for n in ("orc_dump_e4m3", "orc_dump_e8m0", "orc_dump_e2m1"):
            getattr(L, n).argtypes = [_f32p]
        L.orc_matmul_fp8.argtypes = [_f32p, _f32p, _u8p, _vp, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int]
        L.orc_matmul_fp8_n.argtypes = L.orc_matmul_fp8.argtypes + [ctypes.c_int]
        L.orc_matmul_fp4.argtypes = [_f32p, _f32p, _u8p, _u8p, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_matmul_bf16.argtypes = [_f32p, _f32p, _u16p, ctypes.c_int, ctypes.c_int]
        L.orc_argmax.restype = ctypes.c_int
        L.orc_argmax.argtypes = [_f32p, ctypes.c_int]
        L.orc_embed_row.argtypes = [_f32p, ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong,
                                    ctypes.c_int]
        L.orc_swiglu.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        pp = ctypes.POINTER(_u8p)
        L.orc_moe_fp4.argtypes = [_f32p, _f32p, _f32p, pp, pp, pp, pp, pp, pp,
                                  _f32p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_float]
        L.orc_moe_fp4_n.restype = ctypes.c_int
        L.orc_moe_fp4_n.argtypes = [_f32p, _i32p, _f32p, pp, pp, pp, pp, pp, pp, _i32p,
                                    _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_float]
        L.orc_indexer_score.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_topk.restype = ctypes.c_int
        L.orc_topk.argtypes = [_i32p, _f32p, ctypes.c_int, ctypes.c_int]
        L.orc_indexer_offset.argtypes = [_i32p, ctypes.c_int, ctypes.c_int]
        L.orc_indexer_navail.restype = ctypes.c_int
        L.orc_indexer_navail.argtypes = [ctypes.c_int, ctypes.c_int]
        L.orc_window_idxs.restype = ctypes.c_int
        L.orc_window_idxs.argtypes = [_i32p, ctypes.c_int, ctypes.c_int]
        L.orc_sparse_attn.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, _f32p,
                                      _i32p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.orc_rope_apply.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_head_norm_rope.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_float, _f32p, _f32p, ctypes.c_int]
        L.orc_compress_step.restype = ctypes.c_int
        L.orc_compress_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_compress_rope_pos.restype = ctypes.c_int
        L.orc_compress_rope_pos.argtypes = [ctypes.c_int, ctypes.c_int]
        _orc = L
    return _orc


def ref_available():
    return os.path.exists(_REF_PATH)


def ref_moe_available():
    return os.path.exists(_MOE_PATH)


def ref_moe_routed(x, experts, ids, gate_bf16, limit, routed_scale):
    """The reference's own moe() (dsv4_layer.c:369-484) on one token: the
    routed experts `experts` (a list of expert dicts, indexed by id), hash
    routing that selects `ids` (tid2eid of token 0), the BF16 router gate
    [n_exp][hidden] for the weights, and a shared expert of zeros. Returns
    (out, idx, w): moe()'s output -- its routed k-ordered sum plus an exact
    +0.0 per element -- and the selection and weights it used."""
    global _moe
    if _moe is None:
        L = ctypes.CDLL(_MOE_PATH)
        pp = ctypes.POINTER(_u8p)
        L.ref_moe_routed.restype = ctypes.c_int
        L.ref_moe_routed.argtypes = [_f32p, _i32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, pp, pp, pp, pp, pp, pp,
                                     ctypes.POINTER(ctypes.c_int64), _u16p, ctypes.c_float,
                                     ctypes.c_float]
        _moe = L
    x = _f32(x)
    hidden = x.size
    n_exp = len(experts)
    inter = experts[0]["w1"].shape[0]
    ids = np.ascontiguousarray(ids, np.int64)
    topk = ids.size
    gate = np.ascontiguousarray(gate_bf16, np.uint16)
    keep = []

    def arr(name):
        a = (_u8p * n_exp)()
        for e, ex in enumerate(experts):
            v = _u8(ex[name]); keep.append(v); a[e] = _p(v, _u8p)
        return a
    out = np.empty(hidden, np.float32)
    idx = np.empty(topk, np.int32)
    w = np.empty(topk, np.float32)
    rc = _moe.ref_moe_routed(_p(out, _f32p), _p(idx, _i32p), _p(w, _f32p), _p(x, _f32p),
                             hidden, inter, n_exp, topk, arr("w1"), arr("s1"), arr("w3"),
                             arr("s3"), arr("w2"), arr("s2"),
                             ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                             _p(gate, _u16p), limit, routed_scale)
    assert rc == 0
    return out, idx, w


def ref():
    """The compiled reference, or None where it was never built."""
    global _ref
    if _ref is None and ref_available():
        L = ctypes.CDLL(_REF_PATH)
        for n in ("dsv4_matmul_fp8", "dsv4_matmul_fp8_scalar",
                  "dsv4_matmul_fp4", "dsv4_matmul_fp4_scalar"):
            getattr(L, n).argtypes = [_f32p, _f32p, _u8p, _u8p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.dsv4_matmul_fp8_n.argtypes = [_f32p, _f32p, _u8p, _u8p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int]
        for n in ("dsv4_matmul_bf16", "dsv4_matmul_bf16_scalar"):
            getattr(L, n).argtypes = [_f32p, _f32p, _u16p, ctypes.c_int, ctypes.c_int]
        L.dsv4_swiglu.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.dsv4_indexer_score.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int]
        L.dsv4_topk.restype = ctypes.c_int
        L.dsv4_topk.argtypes = [_i32p, _f32p, ctypes.c_int, ctypes.c_int]
        L.dsv4_sparse_attn.argtypes = [_f32p, _f32p, _f32p, _f32p, _i32p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_float, _f32p]
        L.dsv4_rmsnorm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.dsv4_rope_apply.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.dsv4_rope_table.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                      ctypes.c_double, ctypes.c_double]
        L.dsv4_compress_step.restype = ctypes.c_int
        L.dsv4_compress_step.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.dsv4_compress_rope_pos.restype = ctypes.c_int
        L.dsv4_compress_rope_pos.argtypes = [ctypes.c_int, ctypes.c_int]
        _ref = L
    return _ref


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ------------------------------------------------------------------ formats
def dump_e4m3():
    o = np.empty(256, np.float32); lib().orc_dump_e4m3(_p(o, _f32p)); return o


def dump_e8m0():
    o = np.empty(256, np.float32); lib().orc_dump_e8m0(_p(o, _f32p)); return o


def dump_e2m1():
    o = np.empty(16, np.float32); lib().orc_dump_e2m1(_p(o, _f32p)); return o


# ------------------------------------------------------------------ matmuls
def matmul_fp8(x, W, S, blk_r=128, blk_c=128):
    """y = dequant(W) x. S is E8M0 bytes (uint8) or fp32 block scales."""
    W = _u8(W); x = _f32(x)
    out, inn = W.shape
    kind = 1 if np.asarray(S).dtype == np.float32 else 0
    S = np.ascontiguousarray(S)
    if x.ndim == 1:
        y = np.empty(out, np.float32)
        lib().orc_matmul_fp8(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p),
                             S.ctypes.data, kind, inn, out, blk_r, blk_c)
        return y
    nt = x.shape[0]
    y = np.empty((nt, out), np.float32)
    lib().orc_matmul_fp8_n(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p),
                           S.ctypes.data, kind, inn, out, blk_r, blk_c, nt)
    return y


def matmul_bf16(x, W):
    """y = W x for bf16 weights W [out][in] (uint16 bit patterns)."""
    W = np.ascontiguousarray(W, np.uint16); x = _f32(x)
    out, inn = W.shape
    y = np.empty(out, np.float32)
    lib().orc_matmul_bf16(_p(y, _f32p), _p(x, _f32p), W.ctypes.data_as(_u16p), inn, out)
    return y


def argmax(v):
    """The decode loop's greedy pick (dsv4_run.c:471-472)."""
    v = _f32(v)
    return lib().orc_argmax(_p(v, _f32p), v.size)


def embed_row(table, row):
    """dsv4_embed_row: table uint16 (bf16 bits) or float32 [vocab][hidden]."""
    table = np.ascontiguousarray(table)
    wdt = 1 if table.dtype == np.uint16 else 0
    if wdt == 0:
        table = _f32(table)
    dst = np.empty(table.shape[1], np.float32)
    lib().orc_embed_row(_p(dst, _f32p), table.ctypes.data, wdt, int(row), table.shape[1])
    return dst


def matmul_fp4(x, W, S, inn, blk_r=1, blk_c=32):
    W = _u8(W); S = _u8(S); x = _f32(x)
    out = W.shape[0]
    y = np.empty(out, np.float32)
    lib().orc_matmul_fp4(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p), _p(S, _u8p),
                         inn, out, blk_r, blk_c)
    return y


def swiglu(gate, up, limit):
    gate = _f32(gate); up = _f32(up)
    y = np.empty_like(gate)
    lib().orc_swiglu(_p(y, _f32p), _p(gate, _f32p), _p(up, _f32p), gate.size,
                     float(limit))
    return y


def moe_fp4(x, experts, wts, hidden, inter, limit, return_acc=False):
    """experts: list of dicts with w1,s1,w3,s3,w2,s2 (uint8), one per k."""
    x = _f32(x); wts = _f32(wts)
    topk = len(experts)
    keep = []

    def arr(name):
        a = (_u8p * topk)()
        for k, e in enumerate(experts):
            v = _u8(e[name]); keep.append(v); a[k] = _p(v, _u8p)
        return a
    out = np.empty(hidden, np.float32)
    acc = np.empty((topk, hidden), np.float32)
    lib().orc_moe_fp4(_p(out, _f32p), _p(acc, _f32p), _p(x, _f32p),
                      arr("w1"), arr("s1"), arr("w3"), arr("s3"), arr("w2"),
                      arr("s2"), _p(wts, _f32p), topk, hidden, inter,
                      float(limit))
    return (out, acc) if return_acc else out


def moe_fp4_n(X, table, IDX, W, hidden, inter, limit):
    """The routed half of moe_n over a batch: X [nt][hidden], IDX/W
    [nt][topk], table: dict expert id -> expert dict. Returns (out [nt][hidden],
    the distinct experts in first-request order)."""
    X = _f32(X); W = _f32(W)
    IDX = np.ascontiguousarray(IDX, np.int32)
    nt, topk = IDX.shape
    ids = sorted(table)
    pos = {e: i for i, e in enumerate(ids)}
    keep = []

    def arr(name):
        a = (_u8p * len(ids))()
        for i, e in enumerate(ids):
            v = _u8(table[e][name]); keep.append(v); a[i] = _p(v, _u8p)
        return a
    LI = np.ascontiguousarray(np.vectorize(pos.get)(IDX), np.int32)
    out = np.empty((nt, hidden), np.float32)
    uniq = np.empty(nt * topk, np.int32)
    nu = lib().orc_moe_fp4_n(_p(out, _f32p), _p(uniq, _i32p),
                             _p(X, _f32p), arr("w1"), arr("s1"), arr("w3"), arr("s3"),
                             arr("w2"), arr("s2"), _p(LI, _i32p),
                             _p(W, _f32p), nt, topk, hidden, inter, float(limit))
    return out, np.array([ids[i] for i in uniq[:nu]], np.int32)


# ------------------------------------------------------------------ sparse MLA
def indexer_score(q, kv, w, key_stride=None):
    q = _f32(q); kv = _f32(kv); w = _f32(w)
    H, D = q.shape
    stride = D if key_stride is None else key_stride
    n = kv.size // stride
    out = np.empty(n, np.float32)
    lib().orc_indexer_score(_p(out, _f32p), _p(q, _f32p), _p(kv, _f32p),
                            _p(w, _f32p), H, D, n, stride)
    return out


def topk(scores, k):
    scores = _f32(scores)
    kk = max(0, min(k, scores.size))
    idx = np.empty(max(kk, 1), np.int32)
    n = lib().orc_topk(_p(idx, _i32p), _p(scores, _f32p), scores.size, k)
    return idx[:max(n, 0)]


def sparse_attn(q, kv, sink, idxs, scale, d_v=None):
    q = _f32(q); kv = _f32(kv)
    h, d_qk = q.shape
    stride = kv.shape[1]
    d_v = stride if d_v is None else d_v
    idxs = np.ascontiguousarray(idxs, dtype=np.int32)
    sk = None if sink is None else _f32(sink)
    o = np.empty((h, d_v), np.float32)
    lib().orc_sparse_attn(_p(o, _f32p), _p(q, _f32p), _p(kv, _f32p), stride,
                          _p(sk, _f32p), _p(idxs, _i32p), h, d_qk, d_v,
                          idxs.size, float(scale))
    return o


def window_idxs(pos, win):
    idx = np.empty(win, np.int32)
    n = lib().orc_window_idxs(_p(idx, _i32p), pos, win)
    return n, idx


def indexer_navail(pos, ratio):
    return lib().orc_indexer_navail(pos, ratio)


def indexer_offset(idxs, offset):
    idxs = np.array(idxs, dtype=np.int32)
    lib().orc_indexer_offset(_p(idxs, _i32p), idxs.size, offset)
    return idxs


# ------------------------------------------------------------ attention block
def rmsnorm(x, w, eps):
    x = _f32(x); w = _f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(y, _f32p), _p(x, _f32p), _p(w, _f32p), x.size, float(eps))
    return y


def rope_apply(v, rd, cs, sn, pos, inverse=False):
    """v [..., head_dim]: every vector's last rd elements rotated (a copy)."""
    v = np.array(v, dtype=np.float32, order="C")
    cs = _f32(cs); sn = _f32(sn)
    hd = v.shape[-1]
    flat = v.reshape(-1, hd)
    for r in flat:
        lib().orc_rope_apply(_p(r, _f32p), hd, rd, _p(cs, _f32p), _p(sn, _f32p),
                             pos, rd // 2, int(inverse))
    return flat.reshape(v.shape)


def head_norm_rope(q, rd, eps, cs, sn, pos):
    """q [H][hd]: the per-head norm and RoPE of attention() (a copy)."""
    q = np.array(q, dtype=np.float32, order="C")
    cs = _f32(cs); sn = _f32(sn)
    H, hd = q.shape
    lib().orc_head_norm_rope(_p(q, _f32p), H, hd, rd, float(eps), _p(cs, _f32p),
                             _p(sn, _f32p), pos)
    return q


class Compressor:
    """dsv4_compress_step's state for one layer (score state starts at -inf)."""

    def __init__(self, ratio, hd, ape, fn=None):
        ov = ratio == 4
        self.ratio, self.hd, self.width = ratio, hd, (1 + ov) * hd
        self.nslot = (1 + ov) * ratio
        self.ape = _f32(ape)
        self.kv = np.zeros((self.nslot, self.width), np.float32)
        self.sc = np.full((self.nslot, self.width), -np.inf, np.float32)
        self.fn = fn

    def step(self, kv_in, score_in, pos):
        kv_in = _f32(kv_in); score_in = _f32(score_in)
        out = np.zeros(self.hd, np.float32)
        f = self.fn or lib().orc_compress_step
        r = f(_p(out, _f32p), _p(kv_in, _f32p), _p(score_in, _f32p), _p(self.ape, _f32p),
              _p(self.kv, _f32p), _p(self.sc, _f32p), pos, self.ratio, self.hd)
        return out if r == 1 else None


def compress_rope_pos(pos, ratio):
    return lib().orc_compress_rope_pos(pos, ratio)


# ------------------------------------------------- the compiled reference
def ref_rmsnorm(x, w, eps):
    x = _f32(x); w = _f32(w)
    y = np.empty_like(x)
    ref().dsv4_rmsnorm(_p(y, _f32p), _p(x, _f32p), _p(w, _f32p), x.size, float(eps))
    return y


def ref_rope_apply(v, rd, cs, sn, pos, inverse=False):
    v = np.array(v, dtype=np.float32, order="C")
    cs = _f32(cs); sn = _f32(sn)
    hd = v.shape[-1]
    flat = v.reshape(-1, hd)
    for r in flat:
        ref().dsv4_rope_apply(_p(r, _f32p), hd, rd, _p(cs, _f32p), _p(sn, _f32p),
                              pos, rd // 2, int(inverse))
    return flat.reshape(v.shape)


def ref_rope_table(rd, maxpos, orig_ctx, theta, factor=16.0, beta_fast=32.0,
                   beta_slow=1.0):
    """The reference's dsv4_rope_table: cos and sin [maxpos][rd/2]."""
    cs = np.empty((maxpos, rd // 2), np.float32)
    sn = np.empty((maxpos, rd // 2), np.float32)
    ref().dsv4_rope_table(_p(cs, _f32p), _p(sn, _f32p), rd, maxpos, orig_ctx,
                          float(theta), float(factor), float(beta_fast), float(beta_slow))
    return cs, sn


def ref_compressor(ratio, hd, ape):
    return Compressor(ratio, hd, ape, fn=ref().dsv4_compress_step)



def ref_matmul_fp8(x, W, S_e8m0, blk_r=128, blk_c=128, scalar=False):
    W = _u8(W); x = _f32(x); S = _u8(S_e8m0)
    out, inn = W.shape
    y = np.empty(out, np.float32)
    fn = ref().dsv4_matmul_fp8_scalar if scalar else ref().dsv4_matmul_fp8
    fn(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p), _p(S, _u8p), inn, out, blk_r, blk_c)
    return y


def ref_matmul_fp8_n(x, W, S_e8m0, blk_r=128, blk_c=128):
    """The reference's batched dsv4_matmul_fp8_n: x [nt][in] -> y [nt][out]."""
    W = _u8(W); x = _f32(x); S = _u8(S_e8m0)
    out, inn = W.shape
    nt = x.shape[0]
    y = np.empty((nt, out), np.float32)
    ref().dsv4_matmul_fp8_n(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p), _p(S, _u8p),
                            inn, out, blk_r, blk_c, nt)
    return y


def ref_matmul_bf16(x, W, scalar=False):
    W = np.ascontiguousarray(W, np.uint16); x = _f32(x)
    out, inn = W.shape
    y = np.empty(out, np.float32)
    fn = ref().dsv4_matmul_bf16_scalar if scalar else ref().dsv4_matmul_bf16
    fn(_p(y, _f32p), _p(x, _f32p), W.ctypes.data_as(_u16p), inn, out)
    return y


def ref_matmul_fp4(x, W, S, inn, blk_r=1, blk_c=32, scalar=False):
    W = _u8(W); x = _f32(x); S = _u8(S)
    out = W.shape[0]
    y = np.empty(out, np.float32)
    fn = ref().dsv4_matmul_fp4_scalar if scalar else ref().dsv4_matmul_fp4
    fn(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p), _p(S, _u8p), inn, out, blk_r, blk_c)
    return y


def ref_matmul_fp4_n(x, W, S, inn, blk_r=1, blk_c=32):
    """The reference's batched dsv4_matmul_fp4_n (what expert_forward_n's
    dsv4_mmq_n runs for an FP4 matrix): x [nt][in] -> y [nt][out]."""
    W = _u8(W); x = _f32(x); S = _u8(S)
    out = W.shape[0]
    nt = x.shape[0]
    y = np.empty((nt, out), np.float32)
    ref().dsv4_matmul_fp4_n(_p(y, _f32p), _p(x, _f32p), _p(W, _u8p), _p(S, _u8p), inn, out,
                            blk_r, blk_c, nt)
    return y


def ref_swiglu(gate, up, limit):
    gate = _f32(gate); up = _f32(up)
    y = np.empty_like(gate)
    ref().dsv4_swiglu(_p(y, _f32p), _p(gate, _f32p), _p(up, _f32p), gate.size,
                      float(limit))
    return y


def ref_indexer_score(q, kv, w):
    q = _f32(q); kv = _f32(kv); w = _f32(w)
    H, D = q.shape
    n = kv.size // D
    out = np.empty(n, np.float32)
    ref().dsv4_indexer_score(_p(out, _f32p), _p(q, _f32p), _p(kv, _f32p),
                             _p(w, _f32p), H, D, n)
    return out


def ref_topk(scores, k):
    scores = _f32(scores)
    idx = np.empty(max(1, min(k, scores.size)), np.int32)
    n = ref().dsv4_topk(_p(idx, _i32p), _p(scores, _f32p), scores.size, k)
    return idx[:n]


def ref_sparse_attn(q, kv, sink, idxs, scale):
    q = _f32(q); kv = _f32(kv); sink = _f32(sink)
    h, d = q.shape
    idxs = np.ascontiguousarray(idxs, dtype=np.int32)
    o = np.empty((h, d), np.float32)
    scratch = np.empty(h * max(1, idxs.size), np.float32)
    ref().dsv4_sparse_attn(_p(o, _f32p), _p(q, _f32p), _p(kv, _f32p),
                           _p(sink, _f32p), _p(idxs, _i32p), h, d, idxs.size,
                           float(scale), _p(scratch, _f32p))
    return o
