"""Python binding of the MI355X decode backend's C ABI (include/dsv4_gpu.h).

The product is ``lib/libdsv4_gpu.so``: hand-written gfx950 HIP kernels behind
a plain C ABI that is a drop-in for the reference's ``dsv4_cuda_*`` GPU
co-processor (include/dsv4/dsv4_cuda.h:65-99). This module only binds that
ABI with ctypes so the tests and the benchmark can drive it from Python; it
computes nothing itself and has no CPU fallback. If the library is missing,
``lib()`` raises.

Import order matters: PyTorch wheels ship their own HIP runtime under the
same soname (libamdhip64.so.7). Importing torch first makes the dynamic
loader resolve this library's dependency to torch's copy, so there is one
HIP runtime in the process and device pointers from torch tensors are valid
here.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdsv4_gpu.so")
STUB_PATH = os.path.join(HERE, "lib", "libdsv4_gpu_stub.so")

# enum values of include/dsv4_gpu.h and the reference's dsv4.h:92
WF32, WBF16, WFP8, WFP4 = 0, 1, 2, 3
KV_F32, KV_BF16, KV_FP8 = 0, 1, 2
MAX_BATCH = 64

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)
_vp = ctypes.c_void_p
_ci = ctypes.c_int
_cf = ctypes.c_float


class DSV4QMat(ctypes.Structure):
    """Layout of the reference's DSV4QMat (include/dsv4/dsv4.h:208-214)."""
    _fields_ = [("w", _vp), ("s", _vp), ("wdt", _ci), ("rows", _ci),
                ("cols", _ci), ("blk_r", _ci), ("blk_c", _ci)]


class DSV4ExpertW(ctypes.Structure):
    """Layout of the reference's DSV4ExpertW (include/dsv4/dsv4.h:252-255)."""
    _fields_ = [("w1", DSV4QMat), ("w3", DSV4QMat), ("w2", DSV4QMat)]


class AttnCfg(ctypes.Structure):
    """dsv4_gpu_attn_cfg (include/dsv4_gpu.h)."""
    _fields_ = [(n, _ci) for n in ("hidden", "q_lora", "n_heads", "head_dim", "rope_dim",
                                   "window", "ratio", "idx_heads", "idx_dim", "idx_topk",
                                   "o_groups", "o_lora", "max_pos")] + [("rms_eps", _cf)]


class AttnW(ctypes.Structure):
    """dsv4_gpu_attn_w (include/dsv4_gpu.h)."""
    _fields_ = [(n, DSV4QMat) for n in ("wq_a", "wq_b", "wkv", "wo_a", "wo_b", "comp_wkv",
                                        "comp_wgate", "idx_wq_b", "idx_wproj")] + \
               [(n, _vp) for n in ("q_norm", "kv_norm", "sink", "comp_norm", "comp_ape",
                                   "rope_cos", "rope_sin")]


class CkptDims(ctypes.Structure):
    """dsv4_gpu_ckpt_dims (include/dsv4_gpu.h)."""
    _fields_ = [(n, _ci) for n in ("hidden", "q_lora", "n_heads", "head_dim", "o_groups",
                                   "o_lora", "moe_inter", "n_shared", "n_experts",
                                   "index_n_heads", "index_head_dim", "compress_ratio",
                                   "has_indexer")]


class LayerMats(ctypes.Structure):
    """dsv4_gpu_layer_mats (include/dsv4_gpu.h)."""
    _fields_ = [(n, DSV4QMat) for n in ("wq_a", "wq_b", "wkv", "wo_a", "wo_b", "shared_w1",
                                        "shared_w2", "shared_w3", "gate", "comp_wkv",
                                        "comp_wgate", "idx_wq_b", "idx_wproj",
                                        "idx_comp_wkv", "idx_comp_wgate")]


class CkptStats(ctypes.Structure):
    """dsv4_gpu_ckpt_stats (include/dsv4_gpu.h)."""
    _fields_ = [("shards", _ci), ("tensors", ctypes.c_longlong),
                ("matrices", ctypes.c_longlong), ("experts", ctypes.c_longlong),
                ("bytes", ctypes.c_longlong), ("seconds", ctypes.c_double)]


def build():
    """Compile lib/libdsv4_gpu.so (hipcc, gfx950) and the CPU stub."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


_lib = None
_QP = ctypes.POINTER(DSV4QMat)
_EP = ctypes.POINTER(DSV4ExpertW)
_ACP = ctypes.POINTER(AttnCfg)
_AWP = ctypes.POINTER(AttnW)

_SIGS = {
    "dsv4_gpu_available": (_ci, []),
    "dsv4_gpu_set_blocking_sync": (_ci, []),
    "dsv4_gpu_init": (_ci, []),
    "dsv4_gpu_free_vram": (ctypes.c_size_t, []),
    "dsv4_gpu_shutdown": (None, []),
    "dsv4_gpu_upload": (_ci, [_QP]),
    "dsv4_gpu_upload_f32s": (_ci, [_QP]),
    "dsv4_gpu_has": (_ci, [_QP]),
    "dsv4_gpu_mmq": (None, [_vp, _vp, _QP]),
    "dsv4_gpu_mmq_n": (None, [_vp, _vp, _QP, _ci]),
    "dsv4_gpu_fp8_gemv_d": (_ci, [_vp, _vp, _vp, _vp, _ci, _ci, _ci, _vp]),
    "dsv4_gpu_fp8_gemv_n_d": (_ci, [_vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _vp]),
    "dsv4_gpu_fp4_gemv_d": (_ci, [_vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _vp]),
    "dsv4_gpu_bf16_gemv_d": (_ci, [_vp, _vp, _vp, _ci, _ci, _vp]),
    "dsv4_gpu_fp4_gemv_n_d": (_ci, [_vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _ci, _vp]),
    "dsv4_gpu_bf16_gemv_n_d": (_ci, [_vp, _vp, _vp, _ci, _ci, _ci, _vp]),
    "dsv4_gpu_head_argmax": (_ci, [_vp, _QP]),
    "dsv4_gpu_argmax_d": (_ci, [_vp, _vp, _ci, _vp]),
    "dsv4_gpu_embed_row_d": (_ci, [_vp, _vp, _ci, ctypes.c_longlong, _ci, _vp]),
    "dsv4_gpu_dump_e4m3": (_ci, [_vp]),
    "dsv4_gpu_dump_e8m0": (_ci, [_vp]),
    "dsv4_gpu_dump_e2m1": (_ci, [_vp]),
    "dsv4_gpu_dump_fp4_bytes": (_ci, [_vp]),
    "dsv4_gpu_dump_e4m3_scaled": (_ci, [_vp, _ci]),
    "dsv4_gpu_upload_expert": (_ci, [_ci, _ci, _EP]),
    "dsv4_gpu_bind_expert_d": (_ci, [_ci, _ci, _EP]),
    "dsv4_gpu_has_expert": (_ci, [_ci, _ci]),
    "dsv4_gpu_moe_fp4": (_ci, [_vp, _vp, _ci, _vp, _vp, _ci, _ci, _ci, _cf]),
    "dsv4_gpu_moe_fp4_d": (_ci, [_vp, _vp, _ci, _vp, _vp, _ci, _ci, _ci, _cf, _vp]),
    "dsv4_gpu_moe_fp4_n": (_ci, [_vp, _vp, _ci, _vp, _vp, _ci, _ci, _ci, _ci, _cf]),
    "dsv4_gpu_moe_fp4_n_d": (_ci, [_vp, _vp, _ci, _vp, _vp, _ci, _ci, _ci, _ci, _cf, _vp]),
    "dsv4_gpu_moe_fp4_noalloc_d": (_ci, [_vp, _vp, _ci, _vp, _vp, _ci, _ci, _ci, _cf,
                                         _vp]),
    "dsv4_gpu_kv_create": (_vp, [_ci, _ci, _ci]),
    "dsv4_gpu_kv_write_rows": (_ci, [_vp, _ci, _ci, _vp, _vp]),
    "dsv4_gpu_kv_data": (_vp, [_vp]),
    "dsv4_gpu_kv_scales": (_vp, [_vp]),
    "dsv4_gpu_kv_free": (None, [_vp]),
    "dsv4_gpu_indexer_score": (_ci, [_vp, _vp, _vp, _ci, _ci, _vp, _ci, _ci, _ci]),
    "dsv4_gpu_topk": (_ci, [_vp, _vp, _ci, _ci]),
    "dsv4_gpu_indexer_topk": (_ci, [_vp, _vp, _vp, _ci, _ci, _vp, _ci, _ci, _ci, _ci]),
    "dsv4_gpu_sparse_attn": (_ci, [_vp, _vp, _vp, _vp, _vp, _ci, _ci, _ci, _ci, _cf]),
    "dsv4_gpu_indexer_score_d": (_ci, [_vp, _vp, _vp, _ci, _ci, _vp, _vp, _ci, _ci,
                                       _ci, _cf, _vp]),
    "dsv4_gpu_topk_d": (_ci, [_vp, _vp, _ci, _ci, _vp]),
    "dsv4_gpu_sparse_attn_d": (_ci, [_vp, _vp, _vp, _ci, _ci, _ci, _vp, _vp, _ci,
                                     _ci, _ci, _ci, _cf, _vp]),
    "dsv4_gpu_mla_decode_d": (_ci, [_vp, _vp, _vp, _vp, _ci, _ci, _vp, _vp, _ci,
                                    _ci, _ci, _ci, _vp, _vp, _ci, _ci, _ci, _vp,
                                    _ci, _ci, _ci, _cf, _vp]),
    "dsv4_gpu_ckpt_open": (_vp, [ctypes.c_char_p]),
    "dsv4_gpu_ckpt_close": (None, [_vp]),
    "dsv4_gpu_ckpt_has": (_ci, [_vp, ctypes.c_char_p]),
    "dsv4_gpu_ckpt_load_qmat": (_ci, [_vp, ctypes.c_char_p, _ci, _ci, _ci, _QP]),
    "dsv4_gpu_ckpt_load_expert": (_ci, [_vp, _ci, _ci, _ci, _ci, _EP]),
    "dsv4_gpu_ckpt_load_layer": (_ci, [_vp, _vp, _ci, _vp, _vp]),
    "dsv4_gpu_ckpt_stats_get": (_ci, [_vp, _vp]),
    "dsv4_gpu_attn_bind": (_ci, [_ci, _ACP, _AWP]),
    "dsv4_gpu_attn_ready": (_ci, [_ci]),
    "dsv4_gpu_attn_reset": (_ci, [_ci]),
    "dsv4_gpu_attn_step": (_ci, [_vp, _vp, _ci, _ci]),
    "dsv4_gpu_attn_step_d": (_ci, [_vp, _vp, _ci, _ci, _vp]),
}

SYMBOLS = tuple(_SIGS)


def _bind(L):
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def _torch_first():
    try:
        import torch  # noqa: F401  (shares one HIP runtime, see module doc)
    except ImportError:
        pass


def lib(path=None):
    """The loaded HIP backend. Raises if it has not been built."""
    global _lib
    if path is not None:
        _torch_first()
        return _bind(ctypes.CDLL(path))
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "dsv4_gpu: %s is missing; build it with __graft_entry__.build() "
                "(there is no CPU fallback)" % LIB_PATH)
        _torch_first()
        _lib = _bind(ctypes.CDLL(LIB_PATH))
    return _lib


def stub():
    """The CPU-only build of the same ABI (reports no device)."""
    return _bind(ctypes.CDLL(STUB_PATH))


# --------------------------------------------------------------- helpers
def _ptr(a):
    return None if a is None else a.ctypes.data


def init():
    L = lib()
    if not L.dsv4_gpu_available():
        raise RuntimeError("dsv4_gpu: no HIP device")
    if L.dsv4_gpu_init() != 0:
        raise RuntimeError("dsv4_gpu: init failed")
    return L


def qmat(W, S, wdt=WFP8, rows=None, cols=None, blk_r=128, blk_c=128):
    """A DSV4QMat over numpy arrays (the arrays must outlive it)."""
    rows = W.shape[0] if rows is None else rows
    cols = W.shape[1] if cols is None else cols
    return DSV4QMat(W.ctypes.data, None if S is None else S.ctypes.data, wdt, rows, cols,
                    blk_r, blk_c)


def mmq(m, x):
    L = lib()
    y = np.empty(m.rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    L.dsv4_gpu_mmq(_ptr(y), _ptr(x), ctypes.byref(m))
    return y


def mmq_n(m, x):
    L = lib()
    x = np.ascontiguousarray(x, np.float32)
    nt = x.shape[0]
    y = np.empty((nt, m.rows), np.float32)
    L.dsv4_gpu_mmq_n(_ptr(y), _ptr(x), ctypes.byref(m), nt)
    return y


def dump(which):
    L = lib()
    n = {"e4m3": 256, "e8m0": 256, "e2m1": 16, "fp4_bytes": 512}[which]
    out = np.empty(n, np.float32)
    rc = getattr(L, "dsv4_gpu_dump_" + which)(_ptr(out))
    if rc != 0:
        raise RuntimeError("dsv4_gpu: dump %s failed" % which)
    return out


def expert(w1, s1, w3, s3, w2, s2, hidden, inter):
    """DSV4ExpertW over packed FP4 arrays: w1/w3 [inter][hidden/2] with
    s1/s3 [inter][hidden/32], w2 [hidden][inter/2] with s2 [hidden][inter/32]."""
    return DSV4ExpertW(
        DSV4QMat(w1.ctypes.data, s1.ctypes.data, WFP4, inter, hidden, 1, 32),
        DSV4QMat(w3.ctypes.data, s3.ctypes.data, WFP4, inter, hidden, 1, 32),
        DSV4QMat(w2.ctypes.data, s2.ctypes.data, WFP4, hidden, inter, 1, 32))


def moe_fp4(x, layer, idx, w, hidden, inter, limit):
    L = lib()
    out = np.empty(hidden, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    idx = np.ascontiguousarray(idx, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    rc = L.dsv4_gpu_moe_fp4(_ptr(out), _ptr(x), layer, _ptr(idx), _ptr(w),
                            idx.size, hidden, inter, float(limit))
    if rc != 0:
        raise RuntimeError("dsv4_gpu: moe_fp4 failed")
    return out


def moe_fp4_n(X, layer, IDX, Wt, hidden, inter, limit):
    """Batched routed experts (dsv4_gpu_moe_fp4_n): X [nt][hidden], IDX/Wt
    [nt][topk] -> [nt][hidden]."""
    L = lib()
    X = np.ascontiguousarray(X, np.float32)
    IDX = np.ascontiguousarray(IDX, np.int32)
    Wt = np.ascontiguousarray(Wt, np.float32)
    nt, topk = IDX.shape
    out = np.empty((nt, hidden), np.float32)
    rc = L.dsv4_gpu_moe_fp4_n(_ptr(out), _ptr(X), layer, _ptr(IDX), _ptr(Wt), nt, topk,
                              hidden, inter, ctypes.c_float(limit))
    if rc != 0:
        raise RuntimeError("dsv4_gpu: moe_fp4_n failed")
    return out


class KV:
    """A device-resident row store (dsv4_gpu_kv_*)."""

    def __init__(self, n_rows, row_dim, fmt):
        self.L = lib()
        self.h = self.L.dsv4_gpu_kv_create(n_rows, row_dim, fmt)
        if not self.h:
            raise RuntimeError("dsv4_gpu: kv_create failed")
        self.n_rows, self.row_dim, self.fmt = n_rows, row_dim, fmt

    def write(self, row0, rows, scales=None):
        rows = np.ascontiguousarray(rows)
        n = rows.shape[0]
        sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
        if self.L.dsv4_gpu_kv_write_rows(self.h, row0, n, _ptr(rows), _ptr(sc)) != 0:
            raise RuntimeError("dsv4_gpu: kv_write_rows failed")

    def free(self):
        if self.h:
            self.L.dsv4_gpu_kv_free(self.h)
            self.h = None


def indexer_score(q, w, keys, n, row0=0, key_stride=None):
    L = lib()
    q = np.ascontiguousarray(q, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    H, D = q.shape
    out = np.empty(n, np.float32)
    ks = D if key_stride is None else key_stride
    if L.dsv4_gpu_indexer_score(_ptr(out), _ptr(q), _ptr(w), H, D, keys.h, row0,
                                ks, n) != 0:
        raise RuntimeError("dsv4_gpu: indexer_score failed")
    return out


def topk(scores, k):
    L = lib()
    scores = np.ascontiguousarray(scores, np.float32)
    idx = np.empty(max(1, min(k, scores.size)), np.int32)
    n = L.dsv4_gpu_topk(_ptr(idx), _ptr(scores), scores.size, k)
    if n < 0:
        raise RuntimeError("dsv4_gpu: topk failed")
    return idx[:n]


def indexer_topk(q, w, keys, n, k, row0=0, key_stride=None):
    L = lib()
    q = np.ascontiguousarray(q, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    H, D = q.shape
    idx = np.empty(max(1, min(k, n)), np.int32)
    ks = D if key_stride is None else key_stride
    c = L.dsv4_gpu_indexer_topk(_ptr(idx), _ptr(q), _ptr(w), H, D, keys.h, row0,
                                ks, n, k)
    if c < 0:
        raise RuntimeError("dsv4_gpu: indexer_topk failed")
    return idx[:c]


def sparse_attn(q, kv, sink, idxs, scale, d_v=None):
    L = lib()
    q = np.ascontiguousarray(q, np.float32)
    h, d_qk = q.shape
    d_v = kv.row_dim if d_v is None else d_v
    idxs = np.ascontiguousarray(idxs, np.int32)
    sk = None if sink is None else np.ascontiguousarray(sink, np.float32)
    o = np.empty((h, d_v), np.float32)
    if L.dsv4_gpu_sparse_attn(_ptr(o), _ptr(q), kv.h, _ptr(sk), _ptr(idxs), h,
                              d_qk, d_v, idxs.size, float(scale)) != 0:
        raise RuntimeError("dsv4_gpu: sparse_attn failed")
    return o
