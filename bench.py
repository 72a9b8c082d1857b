#!/usr/bin/env python3
"""Benchmark of the MI355X decode hot path.

Headline (the metric's own configuration): the
DeepSeek-scale FP8 trunk GEMV sweep at batch 1 -- 1536x7168, 576x7168,
24576x1536, 7168x16384, 7168x7168 and the 129280x7168 LM head, e4m3 weights
with fp32 128x128 block scales, x ~ N(0,1). One "step" is one decode token's
sweep: the six GEMVs back to back on one stream, every input already resident
in HBM. `value` is achieved HBM GB/s over the sweep (algorithmic bytes /
step time); `ms_per_step` is the time per trunk token (all six shapes).

Timing. Every timed region is a run of launches the GPU executes back to
back, HIP events bracketing exactly the launches timed, with no host launch
latency inside. The headline queues `--warmup` sweeps and then exactly
`--steps` timed sweeps with no synchronisation between them (the host issues
a sweep in far less than its GPU time, so it stays ahead), median of 5
trials. Work the host issues more slowly than the GPU runs it (small
kernels, the attention block) is queued behind a spin kernel sized to the
host's issue time, then warm untimed launches, then the timed ones.

Cold data: one sweep streams 1.15 GB, more than the 256 MB Infinity Cache,
so every matrix has been evicted before it is read again. Per-shape times
rotate distinct copies of the shape (>= 1 GiB in all).

Also reported (`detail`): C1 (4096x4096, rotating 64 copies = 1.07 GB), C3
(MXFP4 routed experts, 8 of 256 resident experts per step = 187 MB, rotated
over the 6 GB expert pool), C4 (the sparse-MLA decode step, rotating 26
copies of the key/KV caches), the BF16 LM head, the batched prefill GEMV and
the attention block at the DeepSeek-V4-Flash shapes.

roofline: the LM-head GEMV (80% of the sweep's bytes), algorithmic bytes per
launch / its average launch time from HIP events on the launch stream.
cpu_baseline: the reference's own CPU path (oracle/_ref, its
dsv4_matmul_fp8 compiled with OpenMP + AVX2) on the same sweep, timed on this
host's cores; `detail.cpu_reference` adds 1-core figures and the reference's
C3, C4 and attention() paths.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

PEAK_GBS = 8000.0
METRIC = ("achieved HBM GB/s (% of peak) for FP8/FP4 decode GEMV; "
          "µs per trunk token")
TRUNK = [(1536, 7168), (576, 7168), (24576, 1536), (7168, 16384), (7168, 7168)]
LM_HEAD = (129280, 7168)


def fp8_bytes(rows, cols):
    """Algorithmic bytes: weights + fp32 block scales + x + y."""
    sr, sc = (rows + 127) // 128, (cols + 127) // 128
    return rows * cols + sr * sc * 4 + cols * 4 + rows * 4


def moe_bytes(hidden, inter, topk):
    per = 2 * inter * (hidden // 2 + hidden // 32) + hidden * (inter // 2 + inter // 32)
    return topk * per + hidden * 2 + hidden * 4 + topk * 8


def rocprof_lm_head_us():
    """The LM-head GEMV's average dispatch duration in the committed rocprof
    summary (profiles/lm_head_kernel_trace.md, `bench.py --only lmhead`
    under rocprofv3 --kernel-trace --stats), or None where it is absent."""
    import re
    try:
        with open(os.path.join(ROOT, "profiles", "lm_head_kernel_trace.md")) as f:
            m = re.search(r"^lm_head_avg_us: ([0-9.]+)", f.read(), re.M)
    except OSError:
        return None
    return float(m.group(1)) if m else None


def lm_head_traffic():
    """HBM bytes per LM-head GEMV launch (FETCH_SIZE + WRITE_SIZE, calibrated
    against a copy of known size), from the committed rocprofv3 summary; None
    when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-detail", action="store_true",
                    help="headline sweep only (skip C1/C3/C4)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c4", "attn", "prefill", "moen", "copy",
                                       "lmhead", "fit", "ckpt"],
                    default=None,
                    help="time one configuration only (for profiling runs); "
                         "'copy' runs a plain 1 GiB device-to-device copy whose "
                         "known size calibrates the FETCH_SIZE/WRITE_SIZE counters")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Bench:
    def __init__(self):
        import numpy as np
        import torch
        import common
        self.np, self.torch, self.common = np, torch, common
        self.dsv4 = common.load_pkg()
        self.L = self.dsv4.init()
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()
        self.sp = self.stream.cuda_stream
        self._cyc_per_ms = None
        self._it = 0

    def t(self, a):
        return self.torch.from_numpy(self.np.ascontiguousarray(a)).to(self.dev)

    def ev(self):
        return self.torch.cuda.Event(enable_timing=True)

    def eager_us(self, go, n, warmup):
        """Per-iteration time of go(i, stream) issued n times eagerly."""
        torch = self.torch
        for i in range(warmup):
            go(i, self.sp)
        torch.cuda.synchronize()
        a, b = self.ev(), self.ev()
        a.record(self.stream)
        for i in range(n):
            go(i, self.sp)
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    def spin(self, ms):
        """A spin kernel of about `ms` on the launch stream (torch's
        clock-based sleep, calibrated once): the launches queued behind it
        are all issued before the first of them runs."""
        torch = self.torch
        if self._cyc_per_ms is None:
            try:
                torch.cuda._sleep(1000)
                a, b = self.ev(), self.ev()
                a.record(self.stream)
                torch.cuda._sleep(1 << 20)
                b.record(self.stream)
                torch.cuda.synchronize()
                self._cyc_per_ms = (1 << 20) / max(a.elapsed_time(b), 1e-3)
            except (AttributeError, RuntimeError):
                self._cyc_per_ms = 0.0
                log("bench: no spin kernel; timed launches start behind the host")
        if self._cyc_per_ms > 0:
            torch.cuda._sleep(int(ms * self._cyc_per_ms))

    def blocked_us(self, go, n, trials=3, warm=None):
        """Per-iteration time of go(i, stream) issued n times back to back,
        median over trials (i keeps counting, so rotations continue). Each
        trial queues a spin kernel long enough for the host to issue
        everything behind it (1.3x the host issue time measured on an
        untimed pass), then `warm` untimed iterations that bring the clocks
        back up after the spin, then the n timed ones between two events.
        Returns (median us, [us per trial])."""
        torch = self.torch
        warm = min(n, 16) if warm is None else warm
        t0 = time.perf_counter()
        for _ in range(n):
            go(self._it, self.sp)
            self._it += 1
        host_ms = (time.perf_counter() - t0) * 1e3 * (n + warm) / n
        torch.cuda.synchronize()
        per = []
        for _ in range(trials):
            self.spin(1.3 * host_ms + 0.2)
            for _ in range(warm):
                go(self._it, self.sp)
                self._it += 1
            a, b = self.ev(), self.ev()
            a.record(self.stream)
            for _ in range(n):
                go(self._it, self.sp)
                self._it += 1
            b.record(self.stream)
            torch.cuda.synchronize()
            per.append(a.elapsed_time(b) * 1e3 / n)
        srt = sorted(per)
        return srt[len(srt) // 2], per

    def graph_us(self, go, n, replays):
        """Per-iteration time with n iterations captured into one HIP graph
        and replayed: no host launch gaps, as a decode loop would run."""
        torch = self.torch
        for i in range(n):                      # settle scratch sizes first
            go(i, self.sp)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            sp = torch.cuda.current_stream().cuda_stream
            for i in range(n):
                go(i, sp)
        g.replay()
        torch.cuda.synchronize()
        a, b = self.ev(), self.ev()
        a.record(self.stream)
        for _ in range(replays):
            g.replay()
        b.record(self.stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / (replays * n)
        del g
        return us

    # --------------------------------------------------------- C2 sweep
    def c2_setup(self):
        np = self.np
        self.c2 = []
        for i, (rows, cols) in enumerate(TRUNK + [LM_HEAD]):
            W, Sf, Se, x = self.common.fp8_problem(i, rows, cols)
            self.c2.append(dict(rows=rows, cols=cols, W=W, Se=Se, x=x,
                                dW=self.t(W), dS=self.t(Sf), dSe=self.t(Se), dx=self.t(x),
                                dy=self.torch.empty(rows, dtype=self.torch.float32,
                                                    device=self.dev)))
        self.torch.cuda.synchronize()

    def c2_launch(self, m, sp=None):
        rc = self.L.dsv4_gpu_fp8_gemv_d(m["dy"].data_ptr(), m["dx"].data_ptr(),
                                        m["dW"].data_ptr(), m["dS"].data_ptr(), 1,
                                        m["rows"], m["cols"],
                                        self.sp if sp is None else sp)
        if rc != 0:
            raise RuntimeError("fp8 gemv launch failed")

    def c2_step(self, i=0, sp=None):
        for m in self.c2:
            self.c2_launch(m, sp)

    def c2_run(self, steps, warmup, trials=5):
        """The headline: per trial, `warmup` untimed sweeps and then exactly
        `steps` timed sweeps, all queued back to back on the stream (the host
        issues a sweep in well under its GPU time, so it stays ahead and the
        GPU never waits on it; the warm sweeps keep the clocks up into the
        timed region); HIP events bracket the timed sweeps. Median over
        `trials` after one untimed trial (ms per sweep, and every timed trial).
        Also, for comparison only:
        the sweeps issued after a synchronisation (eager) and as a HIP graph
        of 10 sweeps replayed 10 times."""
        torch = self.torch
        for i in range(warmup):
            self.c2_step(i)
        torch.cuda.synchronize()
        per = []
        for trial in range(trials + 1):             # the first settles the clocks, untimed
            for i in range(max(1, warmup)):
                self.c2_step(i)
            a, b = self.ev(), self.ev()
            a.record(self.stream)
            for i in range(steps):
                self.c2_step(i)
            b.record(self.stream)
            torch.cuda.synchronize()
            if trial:
                per.append(a.elapsed_time(b) / steps)
        med = sorted(per)[len(per) // 2]
        eager_ms = self.eager_us(self.c2_step, steps, 0) / 1e3
        graph_ms = self.graph_us(self.c2_step, 10, 10) / 1e3
        return med, per, eager_ms, graph_ms

    def c2_shape_run(self, k, reps=3, sfmt=1):
        """One sweep shape alone: distinct copies of it (>= 1 GiB together, so
        each launch reads its weights cold) launched in rotation behind a spin
        kernel; median us per launch over `reps` trials. sfmt 1: the
        configuration's fp32 block scales (the VALU form); 0: the same powers
        of two as E8M0 bytes, the reference's format (the matrix-core form)."""
        torch = self.torch
        m = self.c2[k]
        per_copy = fp8_bytes(m["rows"], m["cols"])
        copies = max(1, min(512, -(-(1 << 30) // per_copy)))
        src = m["dS"] if sfmt else m["dSe"]
        if copies > 1:
            dW = m["dW"].unsqueeze(0).repeat(copies, 1, 1)
            dS = src.unsqueeze(0).repeat(copies, 1, 1)
        else:
            dW, dS = m["dW"].unsqueeze(0), src.unsqueeze(0)
        torch.cuda.synchronize()
        rows, cols = m["rows"], m["cols"]

        def go(i, sp):
            j = i % copies
            if self.L.dsv4_gpu_fp8_gemv_d(m["dy"].data_ptr(), m["dx"].data_ptr(),
                                          dW[j].data_ptr(), dS[j].data_ptr(), sfmt, rows, cols,
                                          sp) != 0:
                raise RuntimeError("fp8 gemv launch failed")
        n = max(2 * copies, 20)
        go(0, self.sp)
        us, _ = self.blocked_us(go, n, reps)
        del dW, dS
        torch.cuda.synchronize()
        return us, copies, n

    # ------------------------------------------------------------ C1
    def c1_run(self, steps, warmup):
        torch, np = self.torch, self.np
        rows = cols = 4096
        W, Sf, Se, x = self.common.fp8_problem(0, rows, cols)
        copies = 64
        dW0, dS0 = self.t(W), self.t(Sf)
        dW = torch.empty((copies, rows, cols), dtype=torch.uint8, device=self.dev)
        dS = torch.empty((copies,) + Sf.shape, dtype=torch.float32, device=self.dev)
        dW[:] = dW0
        dS[:] = dS0
        dx = self.t(x)
        dy = torch.empty(rows, dtype=torch.float32, device=self.dev)

        def go(i, sp):
            j = i % copies
            assert self.L.dsv4_gpu_fp8_gemv_d(dy.data_ptr(), dx.data_ptr(),
                                              dW[j].data_ptr(), dS[j].data_ptr(), 1,
                                              rows, cols, sp) == 0
        eager = self.eager_us(go, max(steps, copies), max(warmup, copies))
        us, _ = self.blocked_us(go, 2 * copies)
        del dW, dS
        return us, eager, fp8_bytes(rows, cols)

    def c1_host_run(self, calls=200):
        """C1 through the reference-compatible host-buffer call dsv4_gpu_mmq:
        x from host memory, y back to host memory, one synchronisation per
        call (H2D + kernel + D2H). 16 resident copies (269 MB) are rotated so
        the weights stay cold. Median wall time per call, in us."""
        import ctypes
        import time
        np = self.np
        rows = cols = 4096
        W, Sf, Se, x = self.common.fp8_problem(0, rows, cols)
        copies = 16
        Ws = [W.copy() for _ in range(copies)]
        ms = [self.dsv4.qmat(Wc, Se, self.dsv4.WFP8, rows, cols, 128, 128) for Wc in Ws]
        for m in ms:
            if self.L.dsv4_gpu_upload(ctypes.byref(m)) != 0:
                raise RuntimeError("upload failed")
        xh = np.ascontiguousarray(x, np.float32)
        yh = np.empty(rows, np.float32)
        px, py = xh.ctypes.data, yh.ctypes.data
        for i in range(2 * copies):
            self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[i % copies]))
        t = []
        for i in range(calls):
            t0 = time.perf_counter()
            self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[i % copies]))
            t.append(time.perf_counter() - t0)
        t.sort()
        self._keep_host = (Ws, ms)
        return t[len(t) // 2] * 1e6

    def host_call_fit(self, reps=200):
        """The per-call cost of the reference-compatible host-buffer call
        dsv4_gpu_mmq (H2D of x, the GEMV, D2H of y, one synchronisation) over
        the reference's own ten shapes (bench/gpu_call.c:60-70, E8M0 scales
        120..134, weights resident), fitted as ms = fixed + MB / bandwidth
        by least squares as bench/gpu_call.c:185-194 does. Two protocols:
        warm, the reference's (one matrix called repeatedly, best of `reps`:
        small matrices then sit in the 256 MB Infinity Cache), and cold
        (distinct resident copies of the shape, >= 512 MiB of them, called
        in rotation; median). Returns the record for `detail`."""
        import ctypes
        np = self.np
        shapes = [(512, 512), (1024, 1024), (2048, 2048), (4096, 1024), (2048, 4096),
                  (4096, 4096), (4096, 8192), (32768, 1024), (8192, 8192), (4096, 16384)]
        rng = np.random.default_rng(20260825)
        rows_out, keep = [], []
        for rows, cols in shapes:
            wb = rows * cols
            sr, sc = (rows + 127) // 128, (cols + 127) // 128
            copies = max(1, -(-(512 << 20) // wb))
            W0 = self.common.fp8_codes(rng, (rows, cols))
            S = (120 + rng.integers(0, 15, size=(sr, sc))).astype(np.uint8)
            x = np.ascontiguousarray(rng.standard_normal(cols).astype(np.float32))
            y = np.empty(rows, np.float32)
            Ws = [W0] + [W0.copy() for _ in range(copies - 1)]
            ms = [self.dsv4.qmat(W, S, self.dsv4.WFP8, rows, cols, 128, 128) for W in Ws]
            for m in ms:
                if self.L.dsv4_gpu_upload(ctypes.byref(m)) != 0:
                    raise RuntimeError("upload failed at %dx%d" % (rows, cols))
            keep.append((Ws, S, ms))
            px, py = x.ctypes.data, y.ctypes.data
            self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[0]))
            warm = []
            for _ in range(reps):
                t0 = time.perf_counter()
                self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[0]))
                warm.append(time.perf_counter() - t0)
            n = max(reps, 2 * copies)
            for i in range(copies):
                self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[i]))
            cold = []
            for i in range(n):
                t0 = time.perf_counter()
                self.L.dsv4_gpu_mmq(py, px, ctypes.byref(ms[i % copies]))
                cold.append(time.perf_counter() - t0)
            cold.sort()
            rows_out.append({"shape": "%dx%d" % (rows, cols), "MB": round(wb / 1048576.0, 3),
                             "warm_best_us": round(min(warm) * 1e6, 2),
                             "cold_median_us": round(cold[len(cold) // 2] * 1e6, 2),
                             "cold_copies": copies})

        def fit(key):
            xs = np.array([r["MB"] for r in rows_out])
            ys = np.array([r[key] / 1e3 for r in rows_out])          # ms
            slope, icept = np.polyfit(xs, ys, 1)
            return {"fixed_us": round(float(icept) * 1e3, 2),
                    "ms_per_MB": round(float(slope), 6),
                    "marginal_GBps": round(1.048576 / float(slope), 1) if slope > 0 else None}
        out = {"shapes": rows_out, "fit_warm_best": fit("warm_best_us"),
               "fit_cold_median": fit("cold_median_us"),
               "reference_published": "ms = 0.0308 + 0.01504 * MB: 31 us fixed, 69.7 GB/s "
                                      "(RTX 5060 Laptop, README.md:460-476)"}
        self._keep_fit = keep        # resident until shutdown: keys are host pointers
        return out

    def ckpt_load_run(self, gib=8, path=None):
        """The checkpoint loader (dsv4_gpu_ckpt_open / _load_qmat: pread into
        pinned staging, one persistent reader thread, copies to HBM) on one
        large synthetic safetensors shard: `gib` GiB of FP8 matrices of
        8192 x 16384 (128 MiB each) with E8M0 scales, written to a file
        first. The file was just written, so it is read from the host page
        cache: this measures the loader's host-to-HBM path, not the storage
        device. Returns the record for `detail`."""
        import ctypes
        import json as _json
        import struct
        import tempfile
        np = self.np
        rows, cols = 8192, 16384
        n = max(1, int(gib * 1024 // 128))
        sb = (rows // 128) * (cols // 128)
        d = tempfile.mkdtemp(prefix="dsv4_ckpt_", dir=path)
        f = os.path.join(d, "model-00001-of-00001.safetensors")
        hdr, off = {}, 0
        for i in range(n):
            hdr["m%d.weight" % i] = {"dtype": "F8_E4M3", "shape": [rows, cols],
                                     "data_offsets": [off, off + rows * cols]}
            off += rows * cols
            hdr["m%d.scale" % i] = {"dtype": "F8_E8M0", "shape": [rows // 128, cols // 128],
                                    "data_offsets": [off, off + sb]}
            off += sb
        j = _json.dumps(hdr, separators=(",", ":")).encode()
        j += b" " * ((-(8 + len(j))) % 8)
        rng = np.random.default_rng(3)
        blob = rng.integers(0, 126, rows * cols, dtype=np.uint8).tobytes()
        sc = np.full(sb, 127, np.uint8).tobytes()
        t0 = time.perf_counter()
        with open(f, "wb") as fh:
            fh.write(struct.pack("<Q", len(j)))
            fh.write(j)
            for i in range(n):
                fh.write(blob)
                fh.write(sc)
        write_s = time.perf_counter() - t0
        L = self.L
        L.dsv4_gpu_ckpt_open.restype = ctypes.c_void_p
        t0 = time.perf_counter()
        ck = L.dsv4_gpu_ckpt_open(f.rsplit("/", 1)[0].encode())
        ms = []
        for i in range(n):
            m = self.dsv4.DSV4QMat()
            if L.dsv4_gpu_ckpt_load_qmat(ctypes.c_void_p(ck), ("m%d" % i).encode(),
                                         self.dsv4.WFP8, rows, cols, ctypes.byref(m)) != 0:
                raise RuntimeError("ckpt load failed at m%d" % i)
            ms.append(m)
        wall = time.perf_counter() - t0
        st = self.dsv4.CkptStats()
        L.dsv4_gpu_ckpt_stats_get(ctypes.c_void_p(ck), ctypes.byref(st))
        L.dsv4_gpu_ckpt_close(ctypes.c_void_p(ck))
        os.unlink(f)
        os.rmdir(d)
        return {"matrices": n, "bytes": int(st.bytes), "file_write_s": round(write_s, 3),
                "load_wall_s": round(wall, 3), "load_GBps_wall": round(st.bytes / wall / 1e9, 2),
                "load_GBps_loader": round(st.bytes / st.seconds / 1e9, 2) if st.seconds else None,
                "source": "host page cache (the shard was just written)"}

    # ------------------------------------------------- BF16 LM head
    def bf16_head_run(self, steps, warmup):
        """The LM head in the reference's own format (BF16 129280x7168,
        dsv4_run.c:467-474), through the BF16 GEMV the dispatch uses for a
        resident BF16 matrix. 1.85 GB: larger than the Infinity Cache, so
        each launch reads it cold."""
        torch = self.torch
        rows, cols = LM_HEAD
        g = torch.Generator(device=self.dev)
        g.manual_seed(7)
        # finite bf16 values: N(0, 1) drawn as float32 and rounded
        W = torch.randn((rows, cols), generator=g, device=self.dev).to(torch.bfloat16)
        dx = torch.randn(cols, generator=g, device=self.dev)
        dy = torch.empty(rows, dtype=torch.float32, device=self.dev)
        torch.cuda.synchronize()

        def go(i, sp):
            assert self.L.dsv4_gpu_bf16_gemv_d(dy.data_ptr(), dx.data_ptr(), W.data_ptr(),
                                               rows, cols, sp) == 0
        eager = self.eager_us(go, max(steps // 4, 4), max(warmup, 2))
        us, _ = self.blocked_us(go, 10)
        del W
        return us, eager, rows * cols * 2 + cols * 4 + rows * 4

    # ------------------------------------------------------- batched (prefill)
    def gemv_n_run(self, rows=7168, cols=7168, nt=64, calls=30, sfmt=0):
        """The batched FP8 GEMV (dsv4_gpu_fp8_gemv_n_d, the k_mmq_fp8_n
        contract: every (row, token) bit-identical to the GEMV) at nt tokens.
        sfmt 0: E8M0 scales (the matrix-core form); 1: fp32 (the VALU form).
        Returns (us per call, GFLOP per call)."""
        torch = self.torch
        W, Sf, Se, x = self.common.fp8_problem(0, rows, cols)
        dW, dS = self.t(W), self.t(Se if sfmt == 0 else Sf)
        dx = torch.randn((nt, cols), device=self.dev)
        dy = torch.empty((nt, rows), device=self.dev)

        def go(i, sp):
            assert self.L.dsv4_gpu_fp8_gemv_n_d(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(),
                                                dS.data_ptr(), sfmt, rows, cols, nt, sp) == 0
        go(0, self.sp)
        us, _ = self.blocked_us(go, calls)
        return us, 2.0 * rows * cols * nt / 1e9

    # ------------------------------------------------------ attention block
    def attn_run(self, steps, warmup, ratio=4, n_layers=4, p0=4096):
        """The attention block (dsv4_gpu_attn_step_d, attention() of
        dsv4_layer.c:213-336 in one call) at the DeepSeek-V4-Flash shapes:
        hidden 4096, 64 heads x 512 (RoPE 64), q_lora 1024, wo_a 8 groups x
        1024, window 128; ratio 4 with the indexer (64 x 128, top 512) or
        ratio 128 (every compressed row). Synthetic FP8 (E8M0 scales) and BF16
        weights of those shapes, random-init. n_layers such layers are bound
        and stepped in turn, so each step reads its layer's weights cold (as a
        decode through the model does); every layer is first decoded to
        position p0, so the ring is full and the compressed rows are p0 /
        ratio (1024 at ratio 4: more than index_topk, so the indexer scores
        and selects on every step). Returns (us per layer step queued behind a
        spin kernel, us per layer step issued from the host, algorithmic
        bytes per layer step)."""
        import ctypes
        np, torch, D, L, C = self.np, self.torch, self.dsv4, self.L, self.common
        hidden, ql, H, hd, rd, win, ol, og = 4096, 1024, 64, 512, 64, 128, 1024, 8
        ih, idd, itop = 64, 128, 512
        has_idx = ratio == 4
        coff = 2 if ratio == 4 else 1
        maxpos = p0 + warmup + 8 * steps + 64
        rng = np.random.default_rng(11)
        keep = []

        def fp8(rows, cols):
            W = C.fp8_codes(rng, (rows, cols))
            S = (127 + rng.integers(-8, -3, size=((rows + 127) // 128,
                                                  (cols + 127) // 128))).astype(np.uint8)
            keep.extend([W, S])
            m = D.DSV4QMat(W.ctypes.data, S.ctypes.data, D.WFP8, rows, cols, 128, 128)
            assert L.dsv4_gpu_upload(ctypes.byref(m)) == 0
            return m, W.nbytes + S.nbytes

        def bf16(rows, cols):
            W = C.bf16_bits((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
            keep.append(W)
            m = D.DSV4QMat(W.ctypes.data, None, D.WBF16, rows, cols, 0, 0)
            assert L.dsv4_gpu_upload(ctypes.byref(m)) == 0
            return m, W.nbytes

        def vec(n, scale=0.1, add=1.0):
            v = (rng.standard_normal(n) * scale + add).astype(np.float32)
            keep.append(v)
            return v.ctypes.data

        half = rd // 2
        th = np.arange(maxpos)[:, None] / (160000.0 ** (np.arange(half) * 2.0 / rd))[None, :]
        cs, sn = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
        keep += [cs, sn]
        layers = list(range(200, 200 + n_layers))
        for lay in layers:
            w = D.AttnW()
            w.wq_a, b0 = fp8(ql, hidden)
            w.wq_b, b1 = fp8(H * hd, ql)
            w.wkv, b2 = fp8(hd, hidden)
            w.wo_a, b3 = fp8(og * ol, H * hd // og)
            w.wo_b, b4 = fp8(hidden, og * ol)
            w.comp_wkv, b5 = bf16(coff * hd, hidden)
            w.comp_wgate, b6 = bf16(coff * hd, hidden)
            mats = b0 + b1 + b2 + b3 + b4 + b5 + b6
            if has_idx:
                w.idx_wq_b, b7 = fp8(ih * idd, ql)
                w.idx_wproj, b8 = bf16(ih, hidden)
                mats += b7 + b8
            w.q_norm, w.kv_norm, w.comp_norm = vec(ql), vec(hd), vec(hd)
            w.sink, w.comp_ape = vec(H, 1.0, 0.0), vec(ratio * coff * hd, 0.5, 0.0)
            w.rope_cos, w.rope_sin = cs.ctypes.data, sn.ctypes.data
            c = D.AttnCfg(hidden=hidden, q_lora=ql, n_heads=H, head_dim=hd, rope_dim=rd,
                          window=win, ratio=ratio, idx_heads=ih if has_idx else 0,
                          idx_dim=idd, idx_topk=itop, o_groups=og, o_lora=ol,
                          max_pos=maxpos, rms_eps=1e-6)
            assert L.dsv4_gpu_attn_bind(lay, ctypes.byref(c), ctypes.byref(w)) == 0
        X = torch.randn((16, hidden), device=self.dev)
        out = torch.empty(hidden, dtype=torch.float32, device=self.dev)
        pos = [0]

        def step(sp):
            p = pos[0]
            for lay in layers:
                assert L.dsv4_gpu_attn_step_d(out.data_ptr(), X[p % 16].data_ptr(), lay, p,
                                              sp) == 0
            pos[0] = p + 1
        while pos[0] < p0:
            step(self.sp)
        torch.cuda.synchronize()
        for _ in range(warmup):
            step(self.sp)
        torch.cuda.synchronize()
        # host-issued (launch gaps included), then behind a spin kernel
        a, b = self.ev(), self.ev()
        a.record(self.stream)
        for _ in range(steps):
            step(self.sp)
        b.record(self.stream)
        torch.cuda.synchronize()
        eager = a.elapsed_time(b) * 1e3 / (steps * n_layers)
        per_pos, _ = self.blocked_us(lambda i, sp: step(sp), steps, 3)
        us = per_pos / n_layers
        avail = p0 // ratio
        take = min(avail, itop) if has_idx else avail
        alg = (mats + 2 * hidden * 4 + (win + take) * hd * 4 +
               (avail * idd * 4 if has_idx else 0))
        for lay in layers:
            L.dsv4_gpu_attn_reset(lay)
        # resident matrices are keyed by host pointer: their host arrays stay
        # allocated for the process, so no later array can reuse an address
        self._attn_keep = getattr(self, "_attn_keep", []) + [keep]
        return us, eager, alg

    # ------------------------------------------------------------ C3
    def c3_run(self, steps, warmup):
        import ctypes
        torch, np = self.torch, self.np
        hidden, inter, topk, n_exp = 7168, 2048, 8, 256
        g = torch.Generator(device=self.dev)
        g.manual_seed(0)
        wb13, sb13 = inter * hidden // 2, inter * hidden // 32
        wb2, sb2 = hidden * inter // 2, hidden * inter // 32
        W13 = torch.randint(0, 256, (n_exp, 2, wb13), dtype=torch.uint8,
                            device=self.dev, generator=g)
        S13 = torch.randint(121, 130, (n_exp, 2, sb13), dtype=torch.uint8,
                            device=self.dev, generator=g)
        W2 = torch.randint(0, 256, (n_exp, wb2), dtype=torch.uint8, device=self.dev,
                           generator=g)
        S2 = torch.randint(121, 130, (n_exp, sb2), dtype=torch.uint8, device=self.dev,
                           generator=g)
        torch.cuda.synchronize()
        D = self.dsv4
        layer = 60
        for e in range(n_exp):
            ew = D.DSV4ExpertW(
                D.DSV4QMat(W13[e, 0].data_ptr(), S13[e, 0].data_ptr(), D.WFP4, inter, hidden, 1, 32),
                D.DSV4QMat(W13[e, 1].data_ptr(), S13[e, 1].data_ptr(), D.WFP4, inter, hidden, 1, 32),
                D.DSV4QMat(W2[e].data_ptr(), S2[e].data_ptr(), D.WFP4, hidden, inter, 1, 32))
            assert self.L.dsv4_gpu_bind_expert_d(layer, e, ctypes.byref(ew)) == 0
        rng = np.random.default_rng(0)
        nsets = 64
        ids = np.stack([rng.permutation(n_exp)[:topk] for _ in range(nsets)]).astype(np.int32)
        ws = np.stack([self.common.router(rng, topk) for _ in range(nsets)])
        d_ids, d_ws = self.t(ids), self.t(ws)
        x = self.common.bf16_round(rng.standard_normal(hidden).astype(np.float32))
        dx = self.t(x)
        do = torch.empty(hidden, dtype=torch.float32, device=self.dev)

        def go(i, sp):
            j = i % nsets
            assert self.L.dsv4_gpu_moe_fp4_d(do.data_ptr(), dx.data_ptr(), layer,
                                             d_ids[j].data_ptr(), d_ws[j].data_ptr(),
                                             topk, hidden, inter, 10.0, sp) == 0
        eager = self.eager_us(go, max(steps, nsets), warmup)
        us, _ = self.blocked_us(go, 2 * nsets)
        del W13, S13, W2, S2
        return us, eager, moe_bytes(hidden, inter, topk)

    # ------------------------------------------------- batched routed experts
    def moe_n_run(self, nts=(1, 4, 16, 64), calls=10):
        """The batched routed experts (dsv4_gpu_moe_fp4_n_d, the routed half
        of moe_n) at C3's expert shape: 256 experts resident, every token of
        the batch routed to 8 of them by a seeded random draw, so experts
        repeat across the batch. Per batch size: us per call, the distinct
        experts it streams, their weight bytes over the time, and the time of
        the same tokens through the single-token call one by one."""
        import ctypes
        torch, np = self.torch, self.np
        hidden, inter, topk, n_exp = 7168, 2048, 8, 256
        g = torch.Generator(device=self.dev)
        g.manual_seed(1)
        wb13, sb13 = inter * hidden // 2, inter * hidden // 32
        wb2, sb2 = hidden * inter // 2, hidden * inter // 32
        W13 = torch.randint(0, 256, (n_exp, 2, wb13), dtype=torch.uint8, device=self.dev,
                            generator=g)
        S13 = torch.randint(121, 130, (n_exp, 2, sb13), dtype=torch.uint8, device=self.dev,
                            generator=g)
        W2 = torch.randint(0, 256, (n_exp, wb2), dtype=torch.uint8, device=self.dev,
                           generator=g)
        S2 = torch.randint(121, 130, (n_exp, sb2), dtype=torch.uint8, device=self.dev,
                           generator=g)
        torch.cuda.synchronize()
        D = self.dsv4
        layer = 61
        for e in range(n_exp):
            ew = D.DSV4ExpertW(
                D.DSV4QMat(W13[e, 0].data_ptr(), S13[e, 0].data_ptr(), D.WFP4, inter, hidden, 1, 32),
                D.DSV4QMat(W13[e, 1].data_ptr(), S13[e, 1].data_ptr(), D.WFP4, inter, hidden, 1, 32),
                D.DSV4QMat(W2[e].data_ptr(), S2[e].data_ptr(), D.WFP4, hidden, inter, 1, 32))
            assert self.L.dsv4_gpu_bind_expert_d(layer, e, ctypes.byref(ew)) == 0
        per_expert = 2 * inter * (hidden // 2 + hidden // 32) + hidden * (inter // 2 + inter // 32)
        rng = np.random.default_rng(3)
        out = {}
        for nt in nts:
            sets = 8
            ids = [np.stack([rng.permutation(n_exp)[:topk] for _ in range(nt)]).astype(np.int32)
                   for _ in range(sets)]
            ws = [np.stack([self.common.router(rng, topk) for _ in range(nt)]) for _ in range(sets)]
            d_ids = [self.t(a) for a in ids]
            d_ws = [self.t(a) for a in ws]
            X = torch.randn((nt, hidden), device=self.dev)
            O = torch.empty((nt, hidden), device=self.dev)

            def go(i, sp):
                j = i % sets
                assert self.L.dsv4_gpu_moe_fp4_n_d(O.data_ptr(), X.data_ptr(), layer,
                                                   d_ids[j].data_ptr(), d_ws[j].data_ptr(), nt,
                                                   topk, hidden, inter, 10.0, sp) == 0

            def one(i, sp):
                j = i % sets
                for t in range(nt):
                    assert self.L.dsv4_gpu_moe_fp4_d(
                        O[t].data_ptr(), X[t].data_ptr(), layer,
                        d_ids[j][t].data_ptr(), d_ws[j][t].data_ptr(), topk, hidden, inter,
                        10.0, sp) == 0
            go(0, self.sp)
            us, _ = self.blocked_us(go, calls)
            us1, _ = self.blocked_us(one, max(2, calls // max(1, nt // 4)))
            uniq = float(np.mean([len(np.unique(a)) for a in ids]))
            out[str(nt)] = {"us": round(us, 3), "distinct_experts": uniq,
                            "GBps_distinct_weights": round(uniq * per_expert / us / 1e3, 1),
                            "token_by_token_us": round(us1, 3)}
        del W13, S13, W2, S2
        return out

    # ------------------------------------------------------------ C4
    def c4_run(self, steps, warmup):
        torch, np = self.torch, self.np
        n, H, D, k, h, dqk, dv = 32768, 16, 128, 2048, 64, 576, 512
        rng = np.random.default_rng(0)
        codes, s, _ = self.common.fp8_keys(rng, n, D)
        kv = self.common.bf16_round(rng.standard_normal((n, dqk)).astype(np.float32)
                                    / np.float32(np.sqrt(dqk)))
        kvb = self.common.bf16_bits(kv).view(np.int16)
        qi = rng.standard_normal((H, D)).astype(np.float32)
        wi = rng.standard_normal(H).astype(np.float32)
        q = rng.standard_normal((h, dqk)).astype(np.float32)
        copies = 26
        d_codes = self.t(codes).unsqueeze(0).repeat(copies, 1, 1)
        d_s = self.t(s).unsqueeze(0).repeat(copies, 1)
        d_kv = self.t(kvb).unsqueeze(0).repeat(copies, 1, 1)
        d_qi, d_wi, d_q = self.t(qi), self.t(wi), self.t(q)
        d_o = torch.empty((h, dv), dtype=torch.float32, device=self.dev)
        d_idx = torch.empty(k, dtype=torch.int32, device=self.dev)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(dqk)))

        def go(i, sp):
            j = i % copies
            assert self.L.dsv4_gpu_mla_decode_d(
                d_o.data_ptr(), d_idx.data_ptr(), d_qi.data_ptr(), d_wi.data_ptr(), H, D,
                d_codes[j].data_ptr(), d_s[j].data_ptr(), self.dsv4.KV_FP8, D, n, k,
                d_q.data_ptr(), d_kv[j].data_ptr(), self.dsv4.KV_BF16, dqk, n, None, h,
                dqk, dv, scale, sp) == 0
        eager = self.eager_us(go, max(steps, copies), max(warmup, copies))
        us, _ = self.blocked_us(go, 2 * copies)
        alg = n * D + n * 4 + k * dqk * 2 + h * dqk * 4 + h * dv * 4 + k * 4 + H * D * 4 + H * 4
        del d_codes, d_s, d_kv
        return us, eager, alg

    # ------------------------------------------------ counter calibration
    def copy_run(self, steps):
        """A plain device-to-device copy of 1 GiB (torch's copy kernel): the
        FETCH_SIZE and WRITE_SIZE counters of a dispatch that reads and writes
        exactly this many bytes give the factor that turns counter readings
        into HBM bytes."""
        torch = self.torch
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device=self.dev)
        a.fill_(1)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        e0, e1 = self.ev(), self.ev()
        e0.record(self.stream)
        for _ in range(max(1, steps)):
            b.copy_(a)
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / max(1, steps), n

    # ------------------------------------------------------ CPU baseline
    def cpu_baseline(self):
        """The compiled reference dsv4_matmul_fp8 (OpenMP + AVX2) over the same
        sweep (E8M0 twin of the power-of-two fp32 scales: identical values),
        repeated until ~10 s of CPU work or 25 sweeps."""
        import oracle
        if not oracle.ref_available():
            return None
        np = self.np
        ys = [np.empty(m["rows"], np.float32) for m in self.c2]
        reps, total = 0, 0.0
        while (total < 10.0 and reps < 25) or reps < 2:
            t0 = time.perf_counter()
            for m in self.c2:
                oracle.ref_matmul_fp8(m["x"], m["W"], m["Se"])
            total += time.perf_counter() - t0
            reps += 1
        per = total / reps
        alg = sum(fp8_bytes(m["rows"], m["cols"]) for m in self.c2)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        return {"value": round(alg / per / 1e9, 3), "unit": "GB/s", "cores": threads,
                "kind": "reference",
                "sample": "the full C2 sweep (5 trunk shapes + LM head, 1.15 GB of "
                          "weights), %d sweeps, %.1f s; %.1f ms per trunk token"
                          % (reps, total, per * 1e3),
                "ms_per_step": round(per * 1e3, 3)}


    def cpu_reference(self):
        """The reference's CPU path beside the device figures, on this host:
        all cores (the OpenMP default) and one core, each a bounded sample.
          c2: one sweep of the six shapes on one core (all cores: cpu_baseline);
          c3: the 8-expert MXFP4 MoE (4 sets of 8 rotated, 748 MB, so the
              weights are cold) -- per expert dsv4_matmul_fp4 w1 / w3,
              dsv4_swiglu (limit 10), dsv4_matmul_fp4 w2, then the k-ordered
              sum (dsv4_layer.c:199-206, :471-475);
          c4: dsv4_indexer_score over 32768 x 128 keys (single-threaded in the
              reference), dsv4_topk at k = 256 of 32768 (O(k^2 n): k = 2048 is
              extrapolated from it, never run), dsv4_sparse_attn over 2048 rows
              of 576 (one width for keys and values, the reference's form), 64
              heads;
          attention(): oracle/_ref/dsv4_attn at the DeepSeek-V4-Flash shapes,
              ratio 4 (CSA, indexer) and 128, positions 4.. of a fresh layer."""
        import ctypes
        import subprocess
        import oracle
        if not oracle.ref_available():
            return None
        np, C = self.np, self.common
        nall = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        try:
            gomp = ctypes.CDLL("libgomp.so.1")
        except OSError:
            gomp = None
        model = "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        out = {"cpu_model": model, "threads_all": nall, "kind": "reference"}

        def best(fn, reps):
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            return min(ts) * 1e3, sum(ts) / len(ts) * 1e3

        def threads(n):
            if gomp is not None:
                gomp.omp_set_num_threads(int(n))
        one = gomp is not None
        # C2 on one core: one sweep
        if one:
            threads(1)
            t0 = time.perf_counter()
            for m in self.c2:
                oracle.ref_matmul_fp8(m["x"], m["W"], m["Se"])
            t = time.perf_counter() - t0
            threads(nall)
            alg = sum(fp8_bytes(m["rows"], m["cols"]) for m in self.c2)
            out["c2_sweep_1core"] = {"ms": round(t * 1e3, 1),
                                     "GBps": round(alg / t / 1e9, 3), "sample": "1 sweep"}
        # C3
        rng = np.random.default_rng(0)
        hidden, inter, topk, nsets = 7168, 2048, 8, 4
        sets = [[C.fp4_expert(rng, hidden, inter) for _ in range(topk)] for _ in range(nsets)]
        x = C.bf16_round(rng.standard_normal(hidden).astype(np.float32))
        wts = C.router(rng, topk)
        turn = [0]

        def c3():
            experts = sets[turn[0] % nsets]
            turn[0] += 1
            acc = np.zeros(hidden, np.float32)
            for k, e in enumerate(experts):
                g = oracle.ref_matmul_fp4(x, e["w1"], e["s1"], hidden)
                u = oracle.ref_matmul_fp4(x, e["w3"], e["s3"], hidden)
                h = oracle.ref_swiglu(g, u, 10.0)
                y = oracle.ref_matmul_fp4(h, e["w2"], e["s2"], inter)
                acc = acc + np.float32(wts[k]) * y
            return acc
        b, m = best(c3, 8)
        out["c3_moe_all_cores"] = {"ms_best": round(b, 2), "ms_mean": round(m, 2),
                                   "GBps": round(moe_bytes(hidden, inter, topk) / b / 1e6, 3),
                                   "sample": "8 calls rotating 4 sets of 8 experts (748 MB)"}
        if one:
            threads(1)
            b, m = best(c3, 2)
            threads(nall)
            out["c3_moe_1core"] = {"ms_best": round(b, 2), "ms_mean": round(m, 2),
                                   "GBps": round(moe_bytes(hidden, inter, topk) / b / 1e6, 3),
                                   "sample": "2 calls, next 2 sets"}
        del sets
        # C4
        n, H, D, h, d = 32768, 16, 128, 64, 576
        codes, ks, deq = C.fp8_keys(rng, n, D)
        qi = rng.standard_normal((H, D)).astype(np.float32)
        wi = rng.standard_normal(H).astype(np.float32)
        sc = [None]

        def score():
            sc[0] = oracle.ref_indexer_score(qi, deq, wi)
        b, _ = best(score, 1)
        out["c4_indexer_score"] = {"ms": round(b, 1), "threads": 1,
                                   "sample": "1 call (the reference's score is single-threaded)"}
        b, _ = best(lambda: oracle.ref_topk(sc[0], 256), 1)
        out["c4_topk"] = {"ms_k256": round(b, 1),
                          "ms_k2048_extrapolated": round(b * 64.0, 0),
                          "sample": "1 call at k = 256 of 32768; k = 2048 scaled by "
                                    "(2048/256)^2 for the O(k^2 n) scan, not run"}
        kv = (rng.standard_normal((n, d)) / np.sqrt(d)).astype(np.float32)
        q = rng.standard_normal((h, d)).astype(np.float32)
        idx = np.sort(rng.permutation(n)[:2048]).astype(np.int32)
        sink = np.full(h, -np.inf, np.float32)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        at = lambda: oracle.ref_sparse_attn(q, kv, sink, idx, scale)  # noqa: E731
        b, m = best(at, 3)
        out["c4_sparse_attn_all_cores"] = {"ms_best": round(b, 2), "ms_mean": round(m, 2),
                                           "sample": "3 calls, h 64, d 576, 2048 rows"}
        if one:
            threads(1)
            b, m = best(at, 2)
            threads(nall)
            out["c4_sparse_attn_1core"] = {"ms_best": round(b, 2), "ms_mean": round(m, 2),
                                           "sample": "2 calls"}
        del kv, deq, codes
        # attention() at the Flash shapes
        exe = os.path.join(ROOT, "oracle", "_ref", "dsv4_attn")
        if os.path.exists(exe):
            for key, ratio, nthr, npos in (("attn_flash_ratio4_all_cores", 4, nall, 12),
                                           ("attn_flash_ratio128_all_cores", 128, nall, 12),
                                           ("attn_flash_ratio4_1core", 4, 1, 6)):
                env = dict(os.environ, OMP_NUM_THREADS=str(nthr))
                try:
                    r = subprocess.run([exe, "--flash", str(npos), str(ratio), "--cpu-only"],
                                       capture_output=True, text=True, timeout=120, env=env)
                except subprocess.TimeoutExpired:
                    continue
                import re
                mm = re.search(r"cpu_ms_per_position (\S+) threads (\d+)", r.stdout)
                if r.returncode == 0 and mm:
                    out[key] = {"ms_per_layer_step": float(mm.group(1)),
                                "threads": int(mm.group(2)),
                                "sample": "positions 4..%d of a fresh layer" % (npos - 1)}
        return out


_STDOUT_FD = None


def quiet_stdout():
    """Send the C library's stdout (its init banner, as the reference's
    dsv4_cuda_init prints one) to stderr, so that stdout carries only the
    JSON line."""
    global _STDOUT_FD
    sys.stdout.flush()
    _STDOUT_FD = os.dup(1)
    os.dup2(2, 1)


def emit(obj):
    import ctypes
    sys.stdout.flush()
    ctypes.CDLL(None).fflush(None)      # C stdio buffers, while fd 1 is stderr
    if _STDOUT_FD is not None:
        os.dup2(_STDOUT_FD, 1)
    print(json.dumps(obj), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU; the multi-GPU sharding of "
              "the decode path is designed (row shards for the GEMVs, expert "
              "shards for the MoE, key shards for the sparse MLA), not launched "
              "(requested --gpus %d)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: WORLD_SIZE > 1 is not supported (one GPU per run)",
              file=sys.stderr)
        sys.exit(2)
    quiet_stdout()
    B = Bench()
    if args.only == "copy":
        us, nbytes = B.copy_run(args.steps)
        emit(({"config": "copy", "bytes_read": nbytes,
                          "bytes_written": nbytes, "us": round(us, 3),
                          "GBps_rw": round(2 * nbytes / us / 1e3, 1)}))
        return
    if args.only == "c2":
        B.c2_setup()
        step_ms, trial_ms, eager_ms, graph_ms = B.c2_run(args.steps, args.warmup)
        per_us = [B.c2_shape_run(k)[0] for k in range(len(B.c2))]
        emit(({"config": "c2", "step_ms": round(step_ms, 4),
               "trials_ms": [round(t, 4) for t in trial_ms],
               "eager_ms": round(eager_ms, 4), "graph_ms": round(graph_ms, 4),
               "per_shape_us": [round(u, 3) for u in per_us]}))
        B.L.dsv4_gpu_shutdown()
        return
    if args.only == "lmhead":
        B.c2_setup()
        us, copies, n = B.c2_shape_run(len(B.c2) - 1)
        a = fp8_bytes(*LM_HEAD)
        emit({"config": "lm_head_fp8_129280x7168", "us": round(us, 3), "copies": copies,
              "launches": n, "GBps": round(a / us / 1e3, 1),
              "frac": round(a / us / 1e3 / PEAK_GBS, 4)})
        B.L.dsv4_gpu_shutdown()
        return
    if args.only == "ckpt":
        emit({"config": "ckpt_load", **B.ckpt_load_run()})
        B.L.dsv4_gpu_shutdown()
        return
    if args.only == "fit":
        emit({"config": "host_call_fit", **B.host_call_fit()})
        B.L.dsv4_gpu_shutdown()
        return
    if args.only == "prefill":
        # the batched matrix-core form unless the caller chose otherwise
        os.environ.setdefault("DSV4_GPU_FP8_MX", "1")
        curve = {}
        for nt in (1, 2, 4, 8, 16, 32, 64):
            us, gf = B.gemv_n_run(nt=nt, calls=20 if nt < 64 else 30)
            curve[str(nt)] = {"us": round(us, 3), "TFLOPs": round(gf / us * 1e3, 2)}
        emit({"config": "prefill_fp8_7168x7168", "by_tokens": curve})
        B.L.dsv4_gpu_shutdown()
        return
    if args.only == "moen":
        emit({"config": "moe_n", "by_tokens": B.moe_n_run()})
        B.L.dsv4_gpu_shutdown()
        return
    if args.only in ("c1", "c3", "c4", "attn"):
        fn = {"c1": B.c1_run, "c3": B.c3_run, "c4": B.c4_run, "attn": B.attn_run}[args.only]
        us, eager, alg = fn(args.steps, args.warmup)
        emit(({"config": args.only, "us": round(us, 3),
                          "eager_us": round(eager, 3),
                          "GBps": round(alg / us / 1e3, 1)}))
        B.L.dsv4_gpu_shutdown()
        return
    log("bench: C2 setup")
    B.c2_setup()
    log("bench: C2 timed sweep, %d steps x 5 trials" % args.steps)
    step_ms, trial_ms, eager_ms, graph_ms = B.c2_run(args.steps, args.warmup)
    shapes = TRUNK + [LM_HEAD]
    algs = [fp8_bytes(r, c) for r, c in shapes]
    alg_step = sum(algs)
    value = alg_step / (step_ms * 1e-3) / 1e9
    per_shape = {}
    per_us = []
    for k, ((r, c), a) in enumerate(zip(shapes, algs)):
        log("bench: C2 shape %dx%d alone" % (r, c))
        us, copies, n = B.c2_shape_run(k)
        per_us.append(us)
        per_shape["%dx%d" % (r, c)] = {"us": round(us, 3), "GBps": round(a / us / 1e3, 1),
                                       "frac": round(a / us / 1e3 / PEAK_GBS, 4),
                                       "copies": copies, "launches": n}
    trunk_us = sum(per_us[:5])
    lm_ms = per_us[5] / 1e3
    lm_gbs = algs[5] / (lm_ms * 1e-3) / 1e9
    traffic = lm_head_traffic()
    rp_us = rocprof_lm_head_us()
    detail = {}

    def rec(us, eager, alg):
        return {"us": round(us, 3), "GBps": round(alg / us / 1e3, 1),
                "frac": round(alg / us / 1e3 / PEAK_GBS, 4),
                "eager_us": round(eager, 3), "algorithmic_bytes": alg}
    if not args.no_detail:
        log("bench: C1")
        detail["c1_fp8_4096x4096"] = rec(*B.c1_run(args.steps, args.warmup))
        log("bench: C1 host-buffer call")
        hus = B.c1_host_run()
        detail["c1_fp8_4096x4096"]["host_call_us"] = round(hus, 2)
        detail["c1_fp8_4096x4096"]["host_call_GBps"] = round(fp8_bytes(4096, 4096) / hus / 1e3, 1)
        log("bench: C3")
        detail["c3_moe_fp4_8of256_7168x2048"] = rec(*B.c3_run(args.steps, args.warmup))
        log("bench: C4")
        detail["c4_sparse_mla_step_32768_top2048"] = rec(*B.c4_run(args.steps, args.warmup))
        log("bench: BF16 LM head")
        detail["lm_head_bf16_129280x7168"] = rec(*B.bf16_head_run(args.steps, args.warmup))
        for form, key in (("0", "c2_e8m0_per_shape"), ("1", "c2_e8m0_per_shape_matrix_core")):
            log("bench: E8M0 shapes (DSV4_GPU_FP8_MX=%s)" % form)
            os.environ["DSV4_GPU_FP8_MX"] = form
            detail[key] = {"form": "VALU (default)" if form == "0" else
                           "matrix core (DSV4_GPU_FP8_MX=1)"}
            for k, ((r, c), a) in enumerate(zip(shapes, algs)):
                us, copies, n = B.c2_shape_run(k, sfmt=0)
                detail[key]["%dx%d" % (r, c)] = {
                    "us": round(us, 3), "GBps": round(a / us / 1e3, 1),
                    "frac": round(a / us / 1e3 / PEAK_GBS, 4)}
        os.environ.pop("DSV4_GPU_FP8_MX", None)
        gf64 = 2.0 * 7168 * 7168 * 64 / 1e9
        for form, key in (("1", "prefill_fp8_7168x7168_nt64"),
                          ("0", "prefill_fp8_7168x7168_nt64_default_form")):
            log("bench: batched prefill GEMV (DSV4_GPU_FP8_MX=%s)" % form)
            os.environ["DSV4_GPU_FP8_MX"] = form
            curve = {}
            for nt in (1, 2, 4, 8, 16, 32, 64):
                us, gf = B.gemv_n_run(nt=nt, calls=20 if nt < 64 else 30)
                curve[str(nt)] = {"us": round(us, 3), "TFLOPs": round(gf / us * 1e3, 2)}
            us = curve["64"]["us"]
            detail[key] = {
                "us": us, "TFLOPs": round(gf64 / us * 1e3, 2),
                "frac_bf16_peak": round(gf64 / us * 1e3 / 2500.0, 4),
                "us_per_token": round(us / 64, 3),
                "scales": "E8M0, " + ("matrix-core form (DSV4_GPU_FP8_MX=1)" if form == "1"
                                      else "VALU form (the default)"),
                "by_tokens": curve}
        os.environ.pop("DSV4_GPU_FP8_MX", None)
        us32, _ = B.gemv_n_run(nt=64, sfmt=1)
        detail["prefill_fp8_7168x7168_nt64_f32_scales"] = {
            "us": round(us32, 3), "TFLOPs": round(gf64 / us32 * 1e3, 2),
            "frac_fp32_peak": round(gf64 / us32 * 1e3 / 157.3, 4), "scales": "fp32 (VALU form)"}
        log("bench: host-buffer call cost fit (dsv4_gpu_mmq, 10 shapes)")
        detail["host_call_fit"] = B.host_call_fit()
        for ratio, name in ((4, "attn_block_flash_csa_ratio4"), (128, "attn_block_flash_hca_ratio128")):
            log("bench: attention block, ratio %d" % ratio)
            detail[name] = rec(*B.attn_run(32, 4, ratio=ratio))
            detail[name]["positions_before"] = 4096
    cpu = None
    if not args.no_cpu:
        log("bench: CPU baseline (compiled reference, host cores)")
        cpu = B.cpu_baseline()
        if not args.no_detail:
            log("bench: CPU reference, C2 on one core, C3, C4, attention()")
            detail["cpu_reference"] = B.cpu_reference()
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy: e4m3 codes uniform over finite, fp32 "
                "scales 2^U{-8..-4}, x ~ N(0,1))",
        "config": {"workload": "C2: DeepSeek-scale FP8 trunk GEMV sweep, batch 1, "
                               "1536x7168 576x7168 24576x1536 7168x16384 7168x7168 "
                               "+ LM head 129280x7168, fp32 128x128 block scales",
                   "batch": 1, "bytes_per_step": alg_step},
        "pct_of_peak": round(100.0 * value / PEAK_GBS, 2),
        "us_per_trunk_token": {"trunk_5_shapes": round(trunk_us, 3),
                               "with_lm_head": round(step_ms * 1e3, 3),
                               "with_lm_head_trials": [round(t * 1e3, 3) for t in trial_ms],
                               "with_lm_head_host_issued": round(eager_ms * 1e3, 3),
                               "with_lm_head_graph_10x10": round(graph_ms * 1e3, 3)},
        "per_shape": per_shape,
        "roofline": {"bound": "hbm", "achieved": round(lm_gbs, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(lm_gbs / PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": "k_fp8_gemv (LM head 129280x7168)",
                     "algorithmic_bytes_per_launch": algs[5],
                     "avg_launch_us": round(lm_ms * 1e3, 3),
                     "rocprof_summary": "profiles/lm_head_kernel_trace.md",
                     "rocprof_avg_us": rp_us,
                     "frac_from_rocprof_avg": (round(algs[5] / rp_us / 1e3 / PEAK_GBS, 4)
                                               if rp_us else None)},
        "cpu_baseline": cpu,
        "detail": detail,
    }
    emit((out))
    B.L.dsv4_gpu_shutdown()


if __name__ == "__main__":
    main()
