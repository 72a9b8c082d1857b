"""Seeded synthetic inputs (the BASELINE.json distributions) and the parity
metrics, shared by the tests and bench.py."""
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "deepseek-v4-in-c_amd")

_pkg = None


def load_pkg():
    global _pkg
    if _pkg is None:
        spec = importlib.util.spec_from_file_location(
            "dsv4_amd", os.path.join(PKG_DIR, "__init__.py"))
        mod = importlib.util.module_from_spec(spec)
        sys.modules["dsv4_amd"] = mod
        spec.loader.exec_module(mod)
        _pkg = mod
    return _pkg


# ------------------------------------------------------------------ data
def fp8_codes(rng, shape):
    """e4m3 bytes uniform over the 254 finite codes (0x7F/0xFF excluded)."""
    v = rng.integers(0, 254, size=shape, dtype=np.uint8)
    v += (v >= 127).astype(np.uint8)
    return v


def fp8_scales(rng, rows, cols, blk=128, continuous=False):
    """Per-128x128-block fp32 scales 2^e, e ~ U{-8..-4} (and the matching
    E8M0 bytes 127+e); or log-uniform in [2^-8, 2^-4] when continuous."""
    sr, sc = (rows + blk - 1) // blk, (cols + blk - 1) // blk
    if continuous:
        f = np.exp2(rng.uniform(-8.0, -4.0, size=(sr, sc))).astype(np.float32)
        return f, None
    e = rng.integers(-8, -3, size=(sr, sc))
    return np.ldexp(1.0, e).astype(np.float32), (127 + e).astype(np.uint8)


def fp8_problem(seed, rows, cols, continuous=False):
    rng = np.random.default_rng(seed)
    W = fp8_codes(rng, (rows, cols))
    Sf, Se = fp8_scales(rng, rows, cols, continuous=continuous)
    x = rng.standard_normal(cols, dtype=np.float32)
    return W, Sf, Se, x


def bf16_round(a):
    """Round f32 to bf16 (RNE) and widen back to f32, exactly."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def bf16_bits(a):
    """bf16 bit patterns of values that are already bf16-exact."""
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def fp4_expert(rng, hidden, inter):
    """One routed expert: nibbles uniform over the 16 codes, E8M0 exponent
    uniform in [-6, 2] per 1x32 block."""
    def mat(rows, cols):
        w = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.int32).astype(np.uint8)
        s = (127 + rng.integers(-6, 3, size=(rows, cols // 32))).astype(np.uint8)
        return w, s
    w1, s1 = mat(inter, hidden)
    w3, s3 = mat(inter, hidden)
    w2, s2 = mat(hidden, inter)
    return dict(w1=w1, s1=s1, w3=w3, s3=s3, w2=w2, s2=s2)


def router(rng, topk):
    z = rng.standard_normal(topk)
    e = np.exp(z - z.max())
    return (e / e.sum()).astype(np.float32)


def e4m3_table():
    import oracle
    return oracle.dump_e4m3()


def fp8_keys(rng, n, d):
    """Indexer keys e4m3(N(0,1)/sqrt(d) / s_row) with a power-of-two fp32
    scale per row; returns (codes, scales, dequantised f32)."""
    v = rng.standard_normal((n, d)).astype(np.float32) / np.float32(np.sqrt(d))
    amax = np.abs(v).max(axis=1)
    s = np.exp2(np.ceil(np.log2(np.maximum(amax, 1e-30) / 448.0))).astype(np.float32)
    tab = e4m3_table()
    finite = np.isfinite(tab)
    vals = tab[finite]
    codes_f = np.nonzero(finite)[0].astype(np.uint8)
    order = np.argsort(vals, kind="stable")
    sv, sc = vals[order], codes_f[order]
    t = (v / s[:, None]).ravel()
    pos = np.clip(np.searchsorted(sv, t), 1, sv.size - 1)
    lo, hi = sv[pos - 1], sv[pos]
    pick = np.where(np.abs(t - lo) <= np.abs(hi - t), pos - 1, pos)
    codes = sc[pick].reshape(n, d)
    deq = (tab[codes] * s[:, None]).astype(np.float32)
    return codes, s, deq


# --------------------------------------------------------------- metrics
def vec_rel_err(got, ref):
    """Worst |got-ref| / max(rms(ref), |got|, |ref|): the vector-scaled metric
    of the reference's GPU gate (tests/unit/test_cuda.c:160-167)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    rms = np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
    s = np.maximum(rms, np.maximum(np.abs(got), np.abs(ref)))
    d = np.abs(got - ref)
    r = np.where(s > 0, d / np.where(s > 0, s, 1), 0.0)
    return float(r.max()) if r.size else 0.0


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def bf16_matrix(rng, shape, scale=1.0):
    """bf16 bit patterns [rows][cols] of N(0, scale^2) values (round to
    nearest even), finite by construction."""
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    u = v.view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r
