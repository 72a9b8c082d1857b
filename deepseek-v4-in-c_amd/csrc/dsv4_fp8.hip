/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_fp8.hip - block-scaled FP8 e4m3 GEMV for batch-1 decode on gfx950.
 *
 * What it computes is dsv4_matmul_fp8 (reference src/core/dsv4_matmul.c:
 * 293-318): y[o] = sum over 128-column blocks of (block dot) * scale(o/128,
 * c/128). It replaces the reference's k_mmq_fp8 (src/cuda/dsv4_cuda.cu:
 * 93-129), which gives each row a 128-thread block and reads one byte per
 * lane per step.
 *
 * APPROACH (bandwidth-bound: ~1 multiply-add per weight byte)
 *   - A row is split over TC threads ("row threads", a power of two up to
 *     64 or a multiple of 64 up to 256); thread j owns the 16-byte chunks
 *     j, j+TC, j+2TC, ... of every row it visits (NCH <= 4 of them), so rows
 *     up to 16384 columns take this path. Consecutive lanes read consecutive 16-byte chunks, so one wave
 *     instruction moves 1 KiB of one row -- fully coalesced.
 *   - The thread's slice of x (NCH x 16 floats) is loaded once into VGPRs and
 *     reused for every row the workgroup visits; workgroups are persistent
 *     over a contiguous range of row tiles, so x is fetched ~once per
 *     workgroup, not once per row.
 *   - A thread works on R rows at once: R*NCH independent 16-byte loads in
 *     flight per lane before any arithmetic.
 *   - Decode is v_cvt_pk_f32_fp8 (exact), 16 fp32 FMAs per chunk, then one
 *     FMA applies the chunk's block scale (each 16-column chunk lies in one
 *     128-column block), accumulating per lane in fp32.
 *   - The TC lane partials of a row are summed by a fixed DPP tree inside a
 *     wave and, when a row spans several waves, in wave order through LDS.
 *
 * DETERMINISM. TC, NCH and the reduction tree are functions of `cols` alone
 * (fp8_geom), so a row's result does not depend on R, the grid size or the
 * rows around it; the batched kernel reuses the same per-row arithmetic and
 * is bit-identical to the GEMV per (row, token).
 *
 * NUMERICS. fp32 inside the lane and in the tree (the reference CPU path
 * accumulates in double); measured against it under the vector-scaled
 * relative metric of tests/unit/test_cuda.c:160-167, bound 1e-5.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <algorithm>
#include <stdlib.h>
#include <type_traits>

namespace {

#include "dsv4_bf16_rows.h"
#include "dsv4_prep_rows.h"

struct Fp8Geom {
    int ch;   /* 16-byte chunks per row                       */
    int tc;   /* threads per row (power of two <= 64, or k*64) */
    int nch;  /* chunks per thread (<= 4)                      */
    int wg;   /* workgroup size                                */
    int rg;   /* rows in flight per workgroup per R            */
};

bool fp8_geom(int cols, Fp8Geom *g)
{
    if (cols <= 0 || (cols & 15)) return false;
    const int ch = cols >> 4;
    int tc, nch;
    if (ch <= 64) {
        tc = 1;
        while (tc < ch) tc <<= 1;
        nch = 1;
    } else {
        tc = 64 * ((ch + 255) / 256);
        nch = (ch + tc - 1) / tc;
    }
    if (tc > 256 || nch > 4) return false;     /* cols <= 16384 */
    g->ch = ch;
    g->tc = tc;
    g->nch = nch;
    g->wg = tc * (256 / tc);
    g->rg = g->wg / tc;
    return true;
}

template <int SF>
__device__ __forceinline__ float ld_scale(const void *S, size_t at)
{
    if (SF == 0) return dec_e8m0(((const uint8_t *)S)[at]);
    return ((const float *)S)[at];
}

/* Dot of 16 decoded weights with 16 activations; 4 interleaved chains. */
/* The chunk's 16 products summed in four chains and a fixed tree, from
 * weights already decoded (dot16f) or from the packed codes (dot16). */
__device__ __forceinline__ float dot16f(const float *w, const float *xr)
{
    float p0 = w[0] * xr[0], p1 = w[1] * xr[1];
    float p2 = w[2] * xr[2], p3 = w[3] * xr[3];
#pragma unroll
    for (int e = 4; e < 16; e += 4) {
        p0 = fmaf(w[e + 0], xr[e + 0], p0);
        p1 = fmaf(w[e + 1], xr[e + 1], p1);
        p2 = fmaf(w[e + 2], xr[e + 2], p2);
        p3 = fmaf(w[e + 3], xr[e + 3], p3);
    }
    return (p0 + p1) + (p2 + p3);
}

__device__ __forceinline__ float dot16(const u32x4 v, const float *xr)
{
    float w[16];
    dec_e4m3x4(v.x, w + 0);
    dec_e4m3x4(v.y, w + 4);
    dec_e4m3x4(v.z, w + 8);
    dec_e4m3x4(v.w, w + 12);
    float p0 = w[0] * xr[0], p1 = w[1] * xr[1];
    float p2 = w[2] * xr[2], p3 = w[3] * xr[3];
#pragma unroll
    for (int e = 4; e < 16; e += 4) {
        p0 = fmaf(w[e + 0], xr[e + 0], p0);
        p1 = fmaf(w[e + 1], xr[e + 1], p1);
        p2 = fmaf(w[e + 2], xr[e + 2], p2);
        p3 = fmaf(w[e + 3], xr[e + 3], p3);
    }
    return (p0 + p1) + (p2 + p3);
}

/* Rows per workgroup are bounded by the LDS that holds the per-wave row
 * partials of rows wider than one wave (at most 4 waves per row). */
constexpr int PART_MAX = 4096;

/* Independent GEMVs of one width in one launch (blockIdx.y = group).
 * Strided: group i reads x + i*x, W + i*w bytes, its scales at S + i*s
 * bytes, and writes y + i*y. Listed (list > 0): group i is matrix Wl[i]
 * (rl[i] rows, scales Sl[i]) into yl[i], all reading the same x. One group
 * with zero strides is the plain GEMV. */
constexpr int FP8_LIST_MAX = 4;
struct Fp8Groups {
    int n = 1;
    long long x = 0, y = 0, w = 0, s = 0;
    int list = 0;
    bool valu = false;                  /* the VALU form even for E8M0 scales */
    const uint8_t *Wl[FP8_LIST_MAX] = {};
    const void *Sl[FP8_LIST_MAX] = {};
    float *yl[FP8_LIST_MAX] = {};
    int rl[FP8_LIST_MAX] = {};
};

/* One step's weights (R rows x NCH chunks) and the block scales of its row
 * block (the R rows of a step lie in one row block: the launcher picks R
 * dividing blk_r, and steps start at multiples of R). Every load is issued
 * unconditionally -- rows past the end read the last row, inactive chunks
 * the last chunk, and their results are discarded -- so no branch stands
 * between the loads and the waits that count them. */
template <int NCH, int R, int SF>
__device__ __forceinline__ void load_step(u32x4 (*wv)[NCH], float *sv, const uint8_t *W,
                                          const void *S, int rbase, int rend, int cols,
                                          int ch, int j, int tc, const int *cb, int sc,
                                          int blk_r)
{
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int r = min(rbase + i, rend - 1);
#pragma unroll
        for (int n = 0; n < NCH; n++) {
            const int c = min(j + n * tc, ch - 1);
            wv[i][n] = ldg16_stream(W + (size_t)r * cols + (size_t)c * 16);
        }
    }
    const int rb = min(rbase, rend - 1) / blk_r;
#pragma unroll
    for (int n = 0; n < NCH; n++) sv[n] = ld_scale<SF>(S, (size_t)rb * sc + cb[n]);
}

/* One workgroup owns the contiguous rows [row0, row0 + rows_per_wg). It walks
 * them in steps of rg*R rows (row group g takes rows g*R .. g*R+R-1 of the
 * step); with PF the next step's weights are in flight while this step's are
 * consumed. Rows that span several waves leave one partial per wave in LDS,
 * summed in wave order after a single barrier at the end. */
/* The GEMV of workgroup (bx, by): rows [bx rows_per_wg, +rows_per_wg) of
 * group or listed matrix by. part: LDS of [waves per row][rows_per_wg]
 * floats, then x (XL), then the norm's weights (NQ). */
template <int NCH, int R, int SF, int PF, int XL, int NQ = 0>
__device__ __forceinline__ void fp8_rows(float *__restrict__ y, const float *__restrict__ x,
                                         const uint8_t *__restrict__ W,
                                         const void *__restrict__ S, int rows, int cols, int sc,
                                         int blk_r, int blk_c, int tc, int rows_per_wg,
                                         const Fp8Groups &gp, int bx, int by, float *part,
                                         const float *__restrict__ nq_w = nullptr,
                                         float nq_eps = 0.0f)
{
    if (gp.list) {
        const int gi = by;
        W = gp.Wl[gi];
        S = gp.Sl[gi];
        y = gp.yl[gi];
        rows = gp.rl[gi];
        if (bx * rows_per_wg >= rows) return;     /* the whole workgroup */
    } else if (gp.n > 1) {
        const size_t gi = by;
        y += gi * gp.y;
        x += gi * gp.x;
        W += gi * gp.w;
        S = (const uint8_t *)S + gi * gp.s;
    }

    const int tid = threadIdx.x;
    const int g = tid / tc;
    const int j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = cols >> 4;
    const int lane = tid & 63;
    const int row0 = bx * rows_per_wg;
    const int rend = min(rows, row0 + rows_per_wg);
    const int nloc = rend - row0;
    const int step_rows = rg * R;
    const int nsteps = (nloc + step_rows - 1) / step_rows;

    float xr[NCH][16];
    int cb[NCH];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        cb[n] = act[n] ? (c * 16) / blk_c : 0;
    }

    u32x4 wv[R][NCH], wn[R][NCH];
    float sv[NCH], sn[NCH];
    if (XL) {
        /* x once per workgroup: the whole workgroup requests all of x (four
         * floats per thread per round, all rounds issued together), then the
         * first step's weights; x lands in LDS and each thread reads its
         * slice from there. Without this, every row group of the workgroup
         * would fetch the same x from L2. */
        float *xs = part + (size_t)(tc > 64 ? tc / 64 : 0) * rows_per_wg;
        constexpr int XR = 4 * NCH;                    /* rounds: cols <= 1024 XR */
        f32x4 xv[XR], nv[NQ ? XR : 1];
        const int nq = cols >> 2;
        /* (NQ: the norm's weights with x, ahead of the weights' requests, and
         * into LDS beside x) */
        float *xw = xs + cols;
#pragma unroll
        for (int q = 0; q < XR; q++) {
            const int i = 4 * min(q * (int)blockDim.x + tid, nq - 1);
            xv[q] = ldf4(x + i);
            if (NQ) nv[q] = ldf4(nq_w + i);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (nsteps > 0)
            load_step<NCH, R, SF>(wv, sv, W, S, row0 + g * R, rend, cols, ch, j, tc, cb, sc,
                                  blk_r);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < XR; q++) {
            const int i = q * (int)blockDim.x + tid;
            if (i < nq) {
                *reinterpret_cast<f32x4 *>(xs + 4 * i) = xv[q];
                if (NQ) *reinterpret_cast<f32x4 *>(xw + 4 * i) = nv[q];
            }
        }
        __syncthreads();
        if (NQ) {
            /* x = w (x inv), the block's weighted RMSNorm (norm_rope_vec,
             * no RoPE) on the workgroup's copy, with its sum of squares in
             * its order: per thread the elements tid, tid + NR_THREADS, ...
             * in order, then block_sum_d (blockDim.x == NR_THREADS) */
            double sq = 0.0;
            for (int i = tid; i < cols; i += NR_THREADS) {
                const double v = (double)xs[i];
                sq += v * v;
            }
            sq = block_sum_d(sq);
            const float inv = (float)(1.0 / sqrt(sq / (double)cols + (double)nq_eps));
            for (int i = tid; i < cols; i += NR_THREADS) {
                const float v = xs[i] * inv;
                xs[i] = xw[i] * v;
            }
            __syncthreads();
        }
#pragma unroll
        for (int n = 0; n < NCH; n++) {
            const int c = min(j + n * tc, ch - 1);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(xs + c * 16 + q * 4);
                xr[n][q * 4 + 0] = v.x; xr[n][q * 4 + 1] = v.y;
                xr[n][q * 4 + 2] = v.z; xr[n][q * 4 + 3] = v.w;
            }
        }
    } else {
#pragma unroll
        for (int n = 0; n < NCH; n++) {
            const int c = j + n * tc;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const f32x4 v = act[n] ? ldf4(x + c * 16 + q * 4) : f32x4{0, 0, 0, 0};
                xr[n][q * 4 + 0] = v.x; xr[n][q * 4 + 1] = v.y;
                xr[n][q * 4 + 2] = v.z; xr[n][q * 4 + 3] = v.w;
            }
        }
        if (nsteps > 0)
            load_step<NCH, R, SF>(wv, sv, W, S, row0 + g * R, rend, cols, ch, j, tc, cb, sc,
                                  blk_r);
    }

    for (int step = 0; step < nsteps; ++step) {
        const int rbase = row0 + step * step_rows + g * R;
        if (PF && step + 1 < nsteps)
            load_step<NCH, R, SF>(wn, sn, W, S, rbase + step_rows, rend, cols, ch, j, tc, cb,
                                  sc, blk_r);

        float acc[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            float a = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const float d = fmaf(dot16(wv[i][n], xr[n]), sv[n], a);
                a = act[n] ? d : a;
            }
            acc[i] = a;
        }

        if (tc <= 64) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = seg_sum_rt(acc[i], tc);
                if (j == tc - 1 && rbase + i < rend) y[rbase + i] = v;
            }
        } else {
            const int w = j >> 6;                  /* wave within the row */
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = seg_sum<64>(acc[i]);
                const int rl = rbase + i - row0;
                if (lane == 63 && rl < nloc) part[w * rows_per_wg + rl] = v;
            }
        }

        if (PF) {
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int n = 0; n < NCH; n++) wv[i][n] = wn[i][n];
#pragma unroll
            for (int n = 0; n < NCH; n++) sv[n] = sn[n];
        } else if (step + 1 < nsteps) {
            load_step<NCH, R, SF>(wv, sv, W, S, rbase + step_rows, rend, cols, ch, j, tc, cb,
                                  sc, blk_r);
        }
    }

    if (tc > 64) {
        __syncthreads();
        const int wpr = tc >> 6;
        for (int rl = tid; rl < nloc; rl += blockDim.x) {
            float s = part[rl];
            for (int w = 1; w < wpr; w++) s += part[w * rows_per_wg + rl];
            y[row0 + rl] = s;
        }
    }
}

template <int NCH, int R, int SF, int PF, int XL>
__global__ void __launch_bounds__(256)
k_fp8_gemv(float *__restrict__ y, const float *__restrict__ x,
           const uint8_t *__restrict__ W, const void *__restrict__ S,
           int rows, int cols, int sc, int blk_r, int blk_c, int tc,
           int rows_per_wg, Fp8Groups gp)
{
    extern __shared__ float part[];     /* [waves per row][rows_per_wg], then x (XL) */
    fp8_rows<NCH, R, SF, PF, XL>(y, x, W, S, rows, cols, sc, blk_r, blk_c, tc, rows_per_wg, gp,
                                 (int)blockIdx.x, (int)blockIdx.y, part);
}

/* Batched: the per-(row, token) arithmetic of k_fp8_gemv with R = 1, looped
 * over tokens in blocks of TB with the row's weight chunks held in VGPRs. */
template <int NCH, int SF>
__global__ void __launch_bounds__(256)
k_fp8_gemv_n(float *__restrict__ y, const float *__restrict__ x,
             const uint8_t *__restrict__ W, const void *__restrict__ S,
             int rows, int cols, int sc, int blk_r, int blk_c, int tc, int nt)
{
    constexpr int TB = 8;
    __shared__ float red[4][TB];

    const int tid = threadIdx.x;
    const int g = tid / tc;
    const int j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = cols >> 4;
    const int wid = tid >> 6, lane = tid & 63;
    const int r = blockIdx.x * rg + g;       /* this row group's row */
    const bool rok = r < rows;

    float wf[NCH][16];                       /* the row's chunks, decoded once */
    float sreg[NCH];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        const u32x4 wv = (act[n] && rok) ? ld16(W + (size_t)r * cols + (size_t)c * 16)
                                         : u32x4{0, 0, 0, 0};
        sreg[n] = (act[n] && rok)
                ? ld_scale<SF>(S, (size_t)(r / blk_r) * sc + (c * 16) / blk_c)
                : 0.0f;
        dec_e4m3x4(wv.x, wf[n] + 0);
        dec_e4m3x4(wv.y, wf[n] + 4);
        dec_e4m3x4(wv.z, wf[n] + 8);
        dec_e4m3x4(wv.w, wf[n] + 12);
    }

    for (int tb = 0; tb < nt; tb += TB) {
        float acc[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) {
            float a = 0.0f;
            if (tb + t < nt) {
                const float *xt = x + (size_t)(tb + t) * cols;
#pragma unroll
                for (int n = 0; n < NCH; n++) {
                    float xr[16];
                    const int c = j + n * tc;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const f32x4 v = act[n] ? ldf4(xt + c * 16 + q * 4)
                                               : f32x4{0, 0, 0, 0};
                        xr[q * 4 + 0] = v.x; xr[q * 4 + 1] = v.y;
                        xr[q * 4 + 2] = v.z; xr[q * 4 + 3] = v.w;
                    }
                    a = fmaf(dot16f(wf[n], xr), sreg[n], a);
                }
            }
            acc[t] = a;
        }
        if (tc <= 64) {
#pragma unroll
            for (int t = 0; t < TB; t++) {
                const float v = seg_sum_rt(acc[t], tc);
                if (j == tc - 1 && rok && tb + t < nt)
                    y[(size_t)(tb + t) * rows + r] = v;
            }
        } else {
            const int wpr = tc >> 6;
#pragma unroll
            for (int t = 0; t < TB; t++) {
                const float v = seg_sum<64>(acc[t]);
                if (lane == 63) red[wid][t] = v;
            }
            __syncthreads();
            if (tid < rg * TB) {
                const int gg = tid / TB, tt = tid - gg * TB;
                const int rr = blockIdx.x * rg + gg;
                float s = red[gg * wpr][tt];
                for (int w = 1; w < wpr; w++) s += red[gg * wpr + w][tt];
                if (rr < rows && tb + tt < nt) y[(size_t)(tb + tt) * rows + rr] = s;
            }
            __syncthreads();
        }
    }
}

/* Any shape the chunked kernel does not take (cols not a multiple of 16, or
 * wider than 16384): one wave per row, one element per lane per step. */
template <int SF>
__global__ void __launch_bounds__(256)
k_fp8_gemv_generic(float *__restrict__ y, const float *__restrict__ x,
                   const uint8_t *__restrict__ W, const void *__restrict__ S,
                   int rows, int cols, int sc, int blk_r, int blk_c, int nt)
{
    const int wpb = blockDim.x >> 6;
    const int r = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const uint8_t *row = W + (size_t)r * cols;
    for (int t = 0; t < nt; t++) {
        const float *xt = x + (size_t)t * cols;
        float a = 0.0f;
        for (int c = lane; c < cols; c += 64) {
            const float s = ld_scale<SF>(S, (size_t)(r / blk_r) * sc + c / blk_c);
            a = fmaf(dec_e4m3(row[c]) * xt[c], s, a);
        }
        const float v = wave_sum(a);
        if (lane == 0) y[(size_t)t * rows + r] = v;
    }
}

int g_cu_count = 0;

int env_int(const char *name, int dflt)
{
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}

int cu_count()
{
    if (!g_cu_count) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        g_cu_count = n;
    }
    return g_cu_count;
}

/* Launch plan of the VALU form: x through LDS or not, the rows each
 * workgroup owns, the grid along x and the dynamic LDS. */
struct Fp8Plan {
    int xl = 0, rows_per_wg = 0, grid = 0;
    size_t lds = 0;
};

Fp8Plan fp8_plan(const Fp8Geom &g, int R, int rows, int cols, int wgs_per_cu, int ngroups)
{
    Fp8Plan p;
    /* x through LDS (one fetch per workgroup instead of one per row group)
     * measured faster on MI355X for narrow rows (24576x1536: 12.2 -> 11.8
     * us) and the widest (7168x16384: 24.8 -> 24.1 us), and within noise
     * or slower between them. */
    p.xl = g.wg == 256 && (cols & 3) == 0 &&
           env_int("DSV4_GPU_FP8_XL", cols <= 2048 || cols >= 16384) != 0;
    const int step_rows = g.rg * R;
    const int nsteps = (rows + step_rows - 1) / step_rows;
    const int want = (wgs_per_cu * cu_count() + ngroups - 1) / ngroups;
    int spw = (nsteps + want - 1) / want;              /* steps per workgroup */
    const int wpr = g.tc > 64 ? g.tc / 64 : 1;
    const int max_spw = PART_MAX / wpr / step_rows;
    if (spw > max_spw) spw = max_spw;
    if (spw < 1) spw = 1;
    p.rows_per_wg = spw * step_rows;
    p.grid = (rows + p.rows_per_wg - 1) / p.rows_per_wg;
    p.lds = (g.tc > 64 ? sizeof(float) * (size_t)wpr * p.rows_per_wg : 0)
          + (p.xl ? sizeof(float) * (size_t)cols : 0);
    return p;
}

template <int NCH, int R, int SF, int PF>
void launch_gemv(const Fp8Geom &g, float *y, const float *x, const uint8_t *W,
                 const void *S, int rows, int cols, int sc, int blk_r,
                 int blk_c, int wgs_per_cu, const Fp8Groups &gp, hipStream_t st)
{
    const Fp8Plan p = fp8_plan(g, R, rows, cols, wgs_per_cu, gp.n);
    const int xl = p.xl, rows_per_wg = p.rows_per_wg, grid = p.grid;
    const size_t lds = p.lds;
    if (xl) {
        static bool opted = false;                  /* x of up to 64 KB + partials */
        if (!opted) {
            (void)dsv4_lds_optin((const void *)k_fp8_gemv<NCH, R, SF, PF, 1>,
                                 dsv4_lds_limit(), "fp8 gemv");
            opted = true;
        }
    }
    if (xl)
        hipLaunchKernelGGL((k_fp8_gemv<NCH, R, SF, PF, 1>), dim3(grid, gp.n), dim3(g.wg), lds,
                           st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, rows_per_wg, gp);
    else
        hipLaunchKernelGGL((k_fp8_gemv<NCH, R, SF, PF, 0>), dim3(grid, gp.n), dim3(g.wg), lds,
                           st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, rows_per_wg, gp);
}

template <int R, int SF, int PF>
void launch_gemv_nch(const Fp8Geom &g, float *y, const float *x,
                     const uint8_t *W, const void *S, int rows, int cols,
                     int sc, int blk_r, int blk_c, int wpc, const Fp8Groups &gp,
                     hipStream_t st)
{
    switch (g.nch) {
    case 1: launch_gemv<1, R, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    case 2: launch_gemv<2, R, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    case 3: launch_gemv<3, R, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    default: launch_gemv<4, R, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    }
}

template <int SF, int PF>
void launch_gemv_r(const Fp8Geom &g, int R, float *y, const float *x,
                   const uint8_t *W, const void *S, int rows, int cols, int sc,
                   int blk_r, int blk_c, int wpc, const Fp8Groups &gp, hipStream_t st)
{
    switch (R) {
    case 1: launch_gemv_nch<1, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    case 2: launch_gemv_nch<2, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    default: launch_gemv_nch<4, SF, PF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st); break;
    }
}

/* Batched with x through LDS (prefill, nt >= 2): a workgroup of 512 threads
 * (rg = 512 / tc row groups) owns the rows [row0, row0 + rows_per_wg) and
 * walks the tokens in blocks of TB, staged in LDS (TB x cols floats) and
 * read by every row group. A row group takes RR rows per step (rb + g,
 * rb + g + rg, ...), decodes their chunks once for the block, and applies
 * each x piece it reads from LDS to all RR rows. Per (row, token) the
 * arithmetic is k_fp8_gemv's (chunk order, scale fma, segment tree, wave
 * partials in wave order), so every result keeps the GEMV's bits. */
template <int NCH, int SF, int TB, int RR>
__global__ void __launch_bounds__(512)
k_fp8_gemv_nl(float *__restrict__ y, const float *__restrict__ x,
              const uint8_t *__restrict__ W, const void *__restrict__ S, int rows, int cols,
              int sc, int blk_r, int blk_c, int tc, int nt, int rows_per_wg)
{
    /* x of the block as [TB][4 quads][ch chunks] 16-byte pieces: a row
     * group's lanes read consecutive pieces (conflict-free), red after */
    extern __shared__ __attribute__((aligned(16))) float xl[];
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = cols >> 4;
    const int wid = tid >> 6, lane = tid & 63;
    const int row0 = blockIdx.x * rows_per_wg;
    const int rend = min(rows, row0 + rows_per_wg);
    float *red = xl + (size_t)TB * cols;
    bool act[NCH];
    int cb[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        cb[n] = (min(c, ch - 1) * 16) / blk_c;
    }
    for (int tb = 0; tb < nt; tb += TB) {
        const int ntb = min(TB, nt - tb);
        __syncthreads();                           /* the previous block's reads */
        {
            const int n4 = (ntb * cols) >> 2;
            const float *xs = x + (size_t)tb * cols;
            for (int i0 = 0; i0 < n4; i0 += 8 * (int)blockDim.x) {
                f32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    v[u] = ldf4(xs + 4 * min(i0 + u * (int)blockDim.x + tid, n4 - 1));
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int i = i0 + u * (int)blockDim.x + tid;
                    if (i < n4) {
                        const int t = (4 * i) / cols, e = 4 * i - t * cols;
                        const int c = e >> 4, q = (e >> 2) & 3;
                        *reinterpret_cast<f32x4 *>(xl + (size_t)t * cols + (size_t)q * ch * 4 +
                                                   c * 4) = v[u];
                    }
                }
            }
        }
        __syncthreads();
        for (int rb = row0; rb < rend; rb += RR * rg) {  /* uniform: every group steps */
            int rr[RR];
            bool rok[RR];
            float wf[RR][NCH][16];
            float sreg[RR][NCH];
#pragma unroll
            for (int k = 0; k < RR; k++) {
                const int r = rb + g + k * rg;
                rok[k] = r < rend;
                rr[k] = rok[k] ? r : rend - 1;
#pragma unroll
                for (int n = 0; n < NCH; n++) {
                    const int c = min(j + n * tc, ch - 1);
                    const u32x4 wv = ld16(W + (size_t)rr[k] * cols + (size_t)c * 16);
                    sreg[k][n] = ld_scale<SF>(S, (size_t)(rr[k] / blk_r) * sc + cb[n]);
                    dec_e4m3x4(wv.x, wf[k][n] + 0);
                    dec_e4m3x4(wv.y, wf[k][n] + 4);
                    dec_e4m3x4(wv.z, wf[k][n] + 8);
                    dec_e4m3x4(wv.w, wf[k][n] + 12);
                }
            }
            float acc[RR][TB];
#pragma unroll
            for (int t = 0; t < TB; t++) {
                float a[RR];
#pragma unroll
                for (int k = 0; k < RR; k++) a[k] = 0.0f;
                const float *xt = xl + (size_t)min(t, ntb - 1) * cols;
#pragma unroll
                for (int n = 0; n < NCH; n++) {
                    const int c = min(j + n * tc, ch - 1);
                    float xr[16];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const f32x4 v =
                            *reinterpret_cast<const f32x4 *>(xt + (size_t)q * ch * 4 + c * 4);
                        xr[q * 4 + 0] = v.x; xr[q * 4 + 1] = v.y;
                        xr[q * 4 + 2] = v.z; xr[q * 4 + 3] = v.w;
                    }
#pragma unroll
                    for (int k = 0; k < RR; k++) {
                        const float d = fmaf(dot16f(wf[k][n], xr), sreg[k][n], a[k]);
                        a[k] = act[n] ? d : a[k];
                    }
                }
#pragma unroll
                for (int k = 0; k < RR; k++) acc[k][t] = a[k];
            }
            if (tc <= 64) {
#pragma unroll
                for (int k = 0; k < RR; k++)
#pragma unroll
                    for (int t = 0; t < TB; t++) {
                        const float v = seg_sum_rt(acc[k][t], tc);
                        if (j == tc - 1 && rok[k] && t < ntb)
                            y[(size_t)(tb + t) * rows + rb + g + k * rg] = v;
                    }
            } else {
                const int wpr = tc >> 6;
#pragma unroll
                for (int k = 0; k < RR; k++)
#pragma unroll
                    for (int t = 0; t < TB; t++) {
                        const float v = seg_sum<64>(acc[k][t]);
                        if (lane == 63) red[(k * 8 + wid) * TB + t] = v;
                    }
                __syncthreads();
                if (tid < RR * rg * TB) {
                    const int k = tid / (rg * TB), rem = tid - k * (rg * TB);
                    const int gg = rem / TB, tt = rem - gg * TB;
                    const int ro = rb + gg + k * rg;
                    const float *rk = red + (size_t)k * 8 * TB;
                    float s = rk[(gg * wpr) * TB + tt];
                    for (int w = 1; w < wpr; w++) s += rk[(gg * wpr + w) * TB + tt];
                    if (ro < rend && tt < ntb) y[(size_t)(tb + tt) * rows + ro] = s;
                }
                __syncthreads();
            }
        }
    }
}

template <int NCH, int SF, int TB>
void launch_gemv_nl(const Fp8Geom &g, float *y, const float *x, const uint8_t *W,
                    const void *S, int rows, int cols, int sc, int blk_r, int blk_c, int nt,
                    hipStream_t st)
{
    constexpr int RR = 2;
    static bool opted = false;
    if (!opted) {
        (void)dsv4_lds_optin((const void *)k_fp8_gemv_nl<NCH, SF, TB, RR>, dsv4_lds_limit(),
                             "fp8 gemv_n");
        opted = true;
    }
    const int step = RR * (512 / g.tc);
    /* about one workgroup per CU: each stages every token block once */
    const int want = cu_count();
    int rpw = (rows + want - 1) / want;
    rpw = (rpw + step - 1) / step * step;
    const int grid = (rows + rpw - 1) / rpw;
    const size_t lds = sizeof(float) * ((size_t)TB * cols + (size_t)RR * 8 * TB);
    hipLaunchKernelGGL((k_fp8_gemv_nl<NCH, SF, TB, RR>), dim3(grid), dim3(512), lds, st, y,
                       x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, nt, rpw);
}

template <int SF, int TB>
void launch_gemv_nl_nch(const Fp8Geom &g, float *y, const float *x, const uint8_t *W,
                        const void *S, int rows, int cols, int sc, int blk_r, int blk_c,
                        int nt, hipStream_t st)
{
    switch (g.nch) {
    case 1: launch_gemv_nl<1, SF, TB>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); break;
    case 2: launch_gemv_nl<2, SF, TB>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); break;
    case 3: launch_gemv_nl<3, SF, TB>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); break;
    default: launch_gemv_nl<4, SF, TB>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); break;
    }
}

/* ---------------------------------------------- batched on the matrix core
 *
 * k_fp8_mfn: the batched GEMV with k_fp8_gemv's bits on v_mfma_f32_16x16x4f32.
 * Measured on the device (an in-bounds probe over 2^21 outputs with normal,
 * wide-exponent, cancelling and subnormal operands, and -0.0 addends), that
 * instruction computes each output as a sequential fmaf chain over its four
 * k in ascending order, starting from C, without flushing subnormals. Each
 * of dot16's four chains (elements c, c+4, c+8, c+12 of a chunk: a product,
 * then three fmaf) is therefore one MFMA with A[row][k] = w[c + 4k],
 * B[k][token] = x[c + 4k] and C = -0.0 (fmaf(a, b, -0.0) == a * b, signed
 * zeros included). The VALU runs the rest of k_fp8_gemv's per-(row, token)
 * arithmetic in its order: (p0 + p1) + (p2 + p3), fmaf with the chunk's
 * scale into row slot j's running sum (chunks j, j + tc, ... in order, from
 * +0.0), and the slots' fixed tree (balanced over aligned blocks within 64
 * slots, then the 64-slot blocks in order). Every (row, token) is therefore
 * bit-identical to the single-token GEMV.
 *
 * Layout. The tc slots of a row are cut into P parts of L slots (L in 16,
 * 32, 64, at most 16 steps per part). A workgroup is 8 waves, 8 row tiles of
 * 16, for one part (blockIdx.y) and one tile of 16 tokens (blockIdx.z). A
 * unit is 4 consecutive slots over every n (NCH steps; step n is the chunks
 * j0 + n tc .. + 3, 64 bytes of each row); the workgroup stages its tokens'
 * x of one unit in LDS (two buffers) while the waves run the unit before it,
 * one barrier per unit, so x arrives spread over the kernel instead of in
 * one burst at its start. Lane (row r, k group g) loads dword g of each of a
 * step's 4 chunks, the A operands of their chains, 4 steps ahead; every load
 * is unconditional (steps past the part read its first chunks, x past the
 * last unit its first unit), so each wait counts only the loads before it.
 * A unit ends in a binary-counter tree. With P = 1 the wave writes y; else
 * its part's subtree goes to scratch, and k_fp8_mfn_join forms the rest of
 * the tree. */
constexpr int MFN_PF = 4;               /* steps of weights in flight         */

/* f(std::integral_constant<int, I>{}) for I = 0 .. N-1, unrolled at compile
 * time (register arrays indexed by I stay in registers) */
template <typename F, int... I>
__device__ __forceinline__ void sfor_seq(F &&f, std::integer_sequence<int, I...>)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f)
{
    sfor_seq(f, std::make_integer_sequence<int, N>{});
}

/* LDS floats per token of one unit's x: NCH chunk groups of 64, padded so
 * that the 16 tokens' B reads of one k group fall in distinct banks */
template <int NCH>
struct MfnDim {
    static constexpr int TP = NCH * 64 + 4;
    static constexpr int BUF = 16 * TP;                 /* floats per buffer */
    static constexpr int XM = (16 * NCH * 16 + 511) / 512;  /* float4 per thread */
    static constexpr int UMAX = 16 / NCH;               /* units per part */
};

template <int SF, bool SC1, int NCH>
__global__ void __launch_bounds__(512)
k_fp8_mfn(float *__restrict__ y, float *__restrict__ part, const float *__restrict__ x,
          const uint8_t *__restrict__ W, const void *__restrict__ S, int rows, int cols,
          int sc, int blk_r, int blk_c, int tc, int L, int nt)
{
    using D = MfnDim<NCH>;
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (blockIdx.x * 8 + w) * 16;
    const int p = blockIdx.y, P = gridDim.y;
    const int t0 = blockIdx.z * 16;
    const int ntok = min(16, nt - t0);
    const int ch = cols >> 4;
    const int r = lane & 15, g = lane >> 4;
    const int wrow0 = min(row0, rows - 1);
    const size_t srow = (size_t)(wrow0 / blk_r) * sc;
    const int U = L >> 2;                      /* units, <= D::UMAX */

    /* unit u's chunk group at n, or -1 past the row (4 chunks wholly in or
     * out, as ch % 4 == 0); units past the part read unit 0's */
    auto group = [&](int u, int n) {
        if (u >= U) u = 0;
        const int c = p * L + 4 * u + n * tc;
        return c < ch ? c : -1;
    };
    /* SC1: blk_c a multiple of 64, so a step's 4 chunks share one scale.
     * The scales' bits are read by vector loads (zv: a zero the compiler
     * cannot see through; a scalar load would be counted with the LDS reads,
     * and each wait for x would then also wait for scales requested steps
     * ahead) and taken into scalar registers at use, where the scalar unit
     * decodes them. The weights are read at a uniform base (the step's
     * chunks of the tile's first row) plus a 32-bit lane offset, so their
     * addresses cost no vector instructions. */
    constexpr int NSR = SC1 ? 1 : 4;
    int zv;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zv));
    const uint32_t loff = (uint32_t)((min(wrow0 + r, rows - 1) - wrow0) * cols + 4 * g);
    const uint8_t *const wt = W + (size_t)wrow0 * cols;
    uint32_t WR[16][4];
    uint32_t SR[16][NSR];
    auto wload = [&](auto kc, int u, int n) {
        constexpr int k = decltype(kc)::value;
        const int c = max(group(u, n), 0);
        const uint8_t *wc = wt + (size_t)c * 16;
#pragma unroll
        for (int q = 0; q < 4; q++)
            WR[k][q] = *reinterpret_cast<const uint32_t *>(wc + loff + 16 * q);
#pragma unroll
        for (int q = 0; q < NSR; q++) {
            const size_t at = srow + ((c + q) * 16) / blk_c + zv;
            SR[k][q] = SF == 0 ? (uint32_t)((const uint8_t *)S)[at] : ((const uint32_t *)S)[at];
        }
    };
    /* the step's scale, uniform: from lane 0 into a scalar register */
    auto scale = [&](uint32_t bits) {
        const uint32_t b = __builtin_amdgcn_readfirstlane(bits);
        return SF == 0 ? dec_e8m0(b) : __uint_as_float(b);
    };
    /* x of unit u for the 16 tokens: piece i = (token, n, float4 of 16) */
    f32x4 XV[D::XM];
    auto xload = [&](int u) {
#pragma unroll
        for (int k = 0; k < D::XM; k++) {
            const int i = min((int)threadIdx.x + 512 * k, 16 * NCH * 16 - 1);
            const int t = i / (NCH * 16), n = (i / 16) % NCH, f = i & 15;
            const int c = max(group(u, n), 0);
            XV[k] = ldf4(x + (size_t)(t0 + min(t, ntok - 1)) * cols + c * 16 + 4 * f);
        }
    };
    auto xstore = [&](float *xb) {
#pragma unroll
        for (int k = 0; k < D::XM; k++) {
            const int i = (int)threadIdx.x + 512 * k;
            if (i < 16 * NCH * 16) {
                const int t = i / (NCH * 16), rem = i - t * (NCH * 16);
                *reinterpret_cast<f32x4 *>(xb + t * D::TP + 4 * rem) = XV[k];
            }
        }
    };

    xload(0);
    __builtin_amdgcn_sched_barrier(0);
    sfor<MFN_PF>([&](auto kc) {
        constexpr int s = decltype(kc)::value;
        wload(std::integral_constant<int, s>{}, s / NCH, s % NCH);
    });
    __builtin_amdgcn_sched_barrier(0);
    xstore(xs);
    __builtin_amdgcn_sched_barrier(0);
    xload(1);
    __syncthreads();

    const f32x4 negz = {-0.0f, -0.0f, -0.0f, -0.0f};
    f32x4 h4, h8, h16, h32, fin;
    h4 = h8 = h16 = h32 = fin = f32x4{0.f, 0.f, 0.f, 0.f};
    sfor<D::UMAX>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        const float *xb = xs + (u & 1) * D::BUF + r * D::TP + 4 * g;
        f32x4 A[4];
#pragma unroll
        for (int q = 0; q < 4; q++) A[q] = f32x4{0.f, 0.f, 0.f, 0.f};
        sfor<NCH>([&](auto nc) {
            constexpr int n = decltype(nc)::value;
            constexpr int s = u * NCH + n;
            if constexpr (s + MFN_PF < 16)
                wload(std::integral_constant<int, s + MFN_PF>{}, (s + MFN_PF) / NCH,
                      (s + MFN_PF) % NCH);
            if (u < U && group(u, n) >= 0) {
                /* the step's four x reads first, then chunk q's MFMAs
                 * ahead of chunk q - 1's additions (each chunk's four chains
                 * take 128 cycles of the matrix core, which covers the
                 * previous chunk's results' latency) */
                f32x4 b[4];
                float f[4][4];
#pragma unroll
                for (int q = 0; q < 4; q++)
                    b[q] = *reinterpret_cast<const f32x4 *>(xb + n * 64 + 16 * q);
#pragma unroll
                for (int q = 0; q < 4; q++) dec_e4m3x4(WR[s][q], f[q]);
                f32x4 pp[2][4];
                auto mm = [&](int q, f32x4 *o) {
                    o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(f[q][0], b[q].x, negz, 0, 0, 0);
                    o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(f[q][1], b[q].y, negz, 0, 0, 0);
                    o[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(f[q][2], b[q].z, negz, 0, 0, 0);
                    o[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(f[q][3], b[q].w, negz, 0, 0, 0);
                };
                float sq[4];
#pragma unroll
                for (int q = 0; q < 4; q++) sq[q] = scale(SR[s][SC1 ? 0 : q]);
                auto va = [&](int q, const f32x4 *o) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float d = (o[0][e] + o[1][e]) + (o[2][e] + o[3][e]);
                        A[q][e] = fmaf(d, sq[q], A[q][e]);
                    }
                };
                mm(0, pp[0]);
                __builtin_amdgcn_sched_barrier(0);
                mm(1, pp[1]);
                __builtin_amdgcn_sched_barrier(0);
                va(0, pp[0]);
                __builtin_amdgcn_sched_barrier(0);
                mm(2, pp[0]);
                __builtin_amdgcn_sched_barrier(0);
                va(1, pp[1]);
                __builtin_amdgcn_sched_barrier(0);
                mm(3, pp[1]);
                __builtin_amdgcn_sched_barrier(0);
                va(2, pp[0]);
                va(3, pp[1]);
            }
        });
        if (u < U) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = (A[0][e] + A[1][e]) + (A[2][e] + A[3][e]);
            /* binary counter over units: unit u's 4-slot sum merges with the
             * held blocks of 4, 8, 16 and 32 slots while bits 0..3 of u are
             * set (u is a compile-time constant here) */
            constexpr bool b0 = u & 1, b1 = u & 2, b2 = u & 4, b3 = u & 8;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (!b0) h4[e] = v[e];
                else {
                    const float s1 = h4[e] + v[e];
                    if (!b1) h8[e] = s1;
                    else {
                        const float s2 = h8[e] + s1;
                        if (!b2) h16[e] = s2;
                        else {
                            const float s3 = h16[e] + s2;
                            if (!b3) h32[e] = s3;
                            else fin[e] = h32[e] + s3;
                        }
                    }
                }
            }
        }
        /* the next unit's x into the other buffer (last read by unit u - 1,
         * which every wave finished before the previous barrier), the one
         * after it requested */
        if (u + 1 < D::UMAX) {
            if (u + 1 < U) xstore(xs + ((u + 1) & 1) * D::BUF);
            __builtin_amdgcn_sched_barrier(0);
            xload(u + 2);
            __syncthreads();
        }
    });
    if (row0 >= rows || r >= ntok) return;
    const f32x4 res = L == 16 ? h16 : L == 32 ? h32 : fin;
    float *dst = P == 1 ? y : part + (size_t)p * nt * rows;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int rr = row0 + 4 * g + e;
        if (rr < rows) dst[(size_t)(t0 + r) * rows + rr] = res[e];
    }
}

/* The rest of the slot tree per (row, token) from the P part subtrees:
 * within each 64-slot block the parts' balanced tree, then the blocks in
 * order (tc <= 32: the parts' tree). */
__global__ void __launch_bounds__(256)
k_fp8_mfn_join(float *__restrict__ y, const float *__restrict__ part, int n, int P, int L,
               int tc)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int pb = tc >= 64 ? 64 / L : P;      /* parts per 64-slot block */
    float out = 0.0f;
    for (int k0 = 0; k0 < P; k0 += pb) {
        float v = part[(size_t)k0 * n + i];
        if (pb == 2) v = v + part[(size_t)(k0 + 1) * n + i];
        else if (pb == 4)
            v = (v + part[(size_t)(k0 + 1) * n + i]) +
                (part[(size_t)(k0 + 2) * n + i] + part[(size_t)(k0 + 3) * n + i]);
        out = k0 == 0 ? v : out + v;
    }
    y[i] = out;
}

/* Slots per part of k_fp8_mfn, or 0 where the VALU batched kernel is the
 * faster one (same bits either way). L is the largest of 64, 32, 16 with L
 * nch <= 64 (at most 16 steps per part) and L <= tc, lowered (more parts,
 * more waves) while fewer than about three waves per SIMD would run. The
 * form is taken from 8 tokens on, and only when it has at least one wave
 * per SIMD: below that its 16-token tiles and its serial walk of a part
 * cost more than they save (us, matrix core / VALU, E8M0: 7168x7168 at 4
 * tokens 39.5 / 25.3, 8 tokens 40.3 / 46.9, 16 tokens 40.5 / 89.4, 64
 * tokens 125.5 / 334.7; 576x7168 (288 waves) at 16 tokens 23.6 / 28.1, at 64
 * tokens 24.7 / 102.7; 24576x1536 at 12 tokens 38.2 / 60.5).
 * DSV4_GPU_MFN_L overrides the slots within the same bounds. */
int mfn_slots(const Fp8Geom &g, int rows, int nt)
{
    int lmax = 64;
    while (lmax > 16 && (lmax * g.nch > 64 || lmax > g.tc)) lmax >>= 1;
    if (lmax * g.nch > 64 || lmax > g.tc || g.tc % lmax) return 0;
    const long long tiles = (long long)((rows + 15) / 16) * ((nt + 15) / 16);
    int L = lmax;
    const int e = env_int("DSV4_GPU_MFN_L", 0);
    if (e) {
        if (!((e == 16 || e == 32 || e == 64) && e <= lmax && g.tc % e == 0)) return 0;
        L = e;
    } else {
        while (L > 16 && tiles * (g.tc / L) < 3 * 4 * (long long)cu_count()) L >>= 1;
        if (nt < 8 || tiles * (g.tc / L) < 4 * (long long)cu_count()) return 0;
    }
    return L;
}

bool mfn_ok(const Fp8Geom &g, int cols, int blk_r, int nt, const float *x)
{
    return env_int("DSV4_GPU_FP8_MFN", 1) != 0 && nt >= 2 && (cols & 63) == 0 &&
           g.tc >= 16 && g.tc <= 256 && (blk_r & 15) == 0 && (((uintptr_t)x) & 15) == 0;
}

size_t mfn_scratch_bytes(int rows, int cols, int nt)
{
    Fp8Geom g;
    if (nt < 2 || !fp8_geom(cols, &g)) return 0;
    const int L = mfn_slots(g, rows, nt);
    if (!L || g.tc / L == 1) return 0;
    return sizeof(float) * (size_t)(g.tc / L) * nt * rows;
}

template <int SF>
int launch_gemv_mfn(const Fp8Geom &g, float *y, const float *x, const uint8_t *W,
                    const void *S, int rows, int cols, int sc, int blk_r, int blk_c, int nt,
                    hipStream_t st, void *scratch)
{
    const int L = mfn_slots(g, rows, nt);
    if (!L) return -1;
    const int P = g.tc / L;
    if (P > 1 && !scratch) return -1;
    bool ok = true;
    auto go = [&](auto kern, size_t lds) {         /* two units of x, <= 33 KB */
        if (lds > 64 * 1024) { ok = false; return; }
        const dim3 grid((rows + 127) / 128, P, (nt + 15) / 16);
        hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, y, (float *)scratch, x, W, S, rows,
                           cols, sc, blk_r, blk_c, g.tc, L, nt);
    };
    const bool sc1 = blk_c % 64 == 0;
    switch (g.nch) {
    case 1: sc1 ? go(k_fp8_mfn<SF, true, 1>, 8 * MfnDim<1>::BUF) : go(k_fp8_mfn<SF, false, 1>, 8 * MfnDim<1>::BUF); break;
    case 2: sc1 ? go(k_fp8_mfn<SF, true, 2>, 8 * MfnDim<2>::BUF) : go(k_fp8_mfn<SF, false, 2>, 8 * MfnDim<2>::BUF); break;
    case 3: sc1 ? go(k_fp8_mfn<SF, true, 3>, 8 * MfnDim<3>::BUF) : go(k_fp8_mfn<SF, false, 3>, 8 * MfnDim<3>::BUF); break;
    default: sc1 ? go(k_fp8_mfn<SF, true, 4>, 8 * MfnDim<4>::BUF) : go(k_fp8_mfn<SF, false, 4>, 8 * MfnDim<4>::BUF); break;
    }
    if (!ok) return -1;
    if (P > 1) {
        const int n = nt * rows;
        hipLaunchKernelGGL(k_fp8_mfn_join, dim3((n + 255) / 256), dim3(256), 0, st, y,
                           (const float *)scratch, n, P, L, g.tc);
    }
    return 0;
}

template <int SF>
void launch_gemv_n(const Fp8Geom &g, float *y, const float *x, const uint8_t *W,
                   const void *S, int rows, int cols, int sc, int blk_r,
                   int blk_c, int nt, hipStream_t st, void *scratch)
{
    if (mfn_ok(g, cols, blk_r, nt, x) &&
        launch_gemv_mfn<SF>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st, scratch) == 0)
        return;
    /* two or more tokens: x through LDS, the largest token block that fits
     * and the tokens fill (8 x 4096, 4 x 7168, 2 x 16384 columns) */
    const size_t cap = dsv4_lds_limit() - 2048;
    if (nt >= 2 && (((uintptr_t)x) & 15) == 0 && g.tc <= 256 && 512 % g.tc == 0) {
        const size_t row4 = sizeof(float) * (size_t)cols;
        if (nt >= 8 && 8 * row4 <= cap) { launch_gemv_nl_nch<SF, 8>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); return; }
        if (nt >= 4 && 4 * row4 <= cap) { launch_gemv_nl_nch<SF, 4>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); return; }
        if (2 * row4 <= cap) { launch_gemv_nl_nch<SF, 2>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st); return; }
    }
    const int grid = (rows + g.rg - 1) / g.rg;
    switch (g.nch) {
    case 1: hipLaunchKernelGGL((k_fp8_gemv_n<1, SF>), dim3(grid), dim3(g.wg), 0, st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, nt); break;
    case 2: hipLaunchKernelGGL((k_fp8_gemv_n<2, SF>), dim3(grid), dim3(g.wg), 0, st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, nt); break;
    case 3: hipLaunchKernelGGL((k_fp8_gemv_n<3, SF>), dim3(grid), dim3(g.wg), 0, st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, nt); break;
    default: hipLaunchKernelGGL((k_fp8_gemv_n<4, SF>), dim3(grid), dim3(g.wg), 0, st, y, x, W, S, rows, cols, sc, blk_r, blk_c, g.tc, nt); break;
    }
}

bool blocking_ok(int blk_r, int blk_c)
{
    return blk_r >= 1 && blk_c >= 16 && (blk_c & 15) == 0;
}

/* Which arithmetic a matrix gets, by its format and shape alone (never by the
 * batch size or by where x lies, so the single-token and batched calls agree
 * bit for bit):
 *   - by default every matrix takes the VALU form of this file, the faster
 *     one at batch 1 on every shape measured (E8M0, cold, us, VALU against
 *     matrix core: 576x7168 4.41 / 8.07, 1536x7168 6.04 / 8.44, 24576x1536
 *     10.03 / 11.27, 7168x7168 11.90 / 12.92, 7168x16384 21.58 / 23.85, LM
 *     head 140.4 / 142.2, 2048x4096 4.77 / 6.68, 4096x2048 5.05 / 6.40);
 *   - DSV4_GPU_FP8_MX=1 sends E8M0-scaled matrices the matrix-core form
 *     (dsv4_fp8_mx.hip), single token and batched alike: slower at batch 1,
 *     much faster batched (7168x7168 at 64 tokens 63.9 against 335.2 us),
 *     for prefill-heavy work;
 *   - shapes neither chunked kernel takes run the generic kernel.
 * The chunked forms need x and W 16-byte aligned; a call that breaks that
 * is refused rather than sent to another arithmetic (chunked_ok). */
bool mx_form(int sfmt, int cols, int blk_r, int blk_c)
{
    return env_int("DSV4_GPU_FP8_MX", 0) != 0 && dsv4_fp8_mx_ok(sfmt, cols, blk_r, blk_c);
}

/* x and W of a chunked-form call are 16-byte aligned; else -1 with a
 * message (the host-buffer entry points stage x aligned, and the
 * residency keeps W as allocated, so only a caller's device pointer can
 * break this). */
int chunked_ok(const float *x, const uint8_t *W, const char *what)
{
    if ((((uintptr_t)x | (uintptr_t)W) & 15) == 0) return 0;
    DSV4_ERR("%s: x (%p) and W (%p) must be 16-byte aligned", what, (const void *)x,
             (const void *)W);
    return -1;
}

/* The VALU form's launch parameters for a matrix of rows x cols: R rows per
 * thread per step (at most blk_r's largest power-of-two divisor up to 4),
 * the next step prefetched or not, workgroups per CU. None of these changes
 * a row's arithmetic, and the environment can override each. The rule, from
 * sweeps over the C1/C2 and attention-block shapes on MI355X (R in 1, 2, 4;
 * prefetch on/off; x through LDS or not; 1-8 workgroups per CU; cold, us):
 *   - two workgroups per CU (four when rows are narrow, cols < 4096);
 *   - rows of 16384 columns with fp32 scales: one row per step with the
 *     next prefetched (7168x16384: 21.7-22.2 -> 21.1-21.3); with E8M0
 *     scales the base below (21.2-21.4 against 22.4-22.5 for one row);
 *   - more than 4096 rows: two rows per step without prefetch, unless that
 *     grid leaves its last round of workgroups short, so that some CUs get
 *     fewer than others, while one row per step fills it (7168x7168: 448
 *     workgroups at two rows, 512 at one; 12.0 -> 11.5). The LM head keeps
 *     two (505 workgroups; one row per step measured 147 against 137.5);
 *   - at most 4096 rows of at least 4096 columns: one row per step without
 *     prefetch where that grid is one round of workgroups (1024x4096 4.4 ->
 *     3.8, 512x4096 4.2 -> 3.6, either scale format), or, with E8M0 scales,
 *     where its rounds are full (4096x8192 9.9 -> 9.1, 4096x4096 6.2 ->
 *     6.1; with fp32 scales, whose step loads four bytes of scale per
 *     chunk, 9.5 either way and 6.1 against 6.2 for two rows);
 *     else four rows per step without prefetch where only that grid is
 *     full (1536x7168: 384 workgroups at two rows, 192 at four; 5.9 ->
 *     5.7); otherwise, and for narrower rows, two rows per step with the
 *     next prefetched (576x7168: 4.3 at two rows, 4.6 at one, whose 288
 *     workgroups spill onto 32 CUs).
 * tuned = false keeps the base rule (two rows; prefetch where rows <= 4096)
 * for the attention block's combined launches, which are built for it. */
struct Fp8Valu {
    int R, pf, wpc;
};

Fp8Valu fp8_valu(int rows, int cols, int blk_r, int sfmt, bool tuned = true)
{
    Fp8Valu v;
    v.wpc = env_int("DSV4_GPU_FP8_WPC", cols >= 4096 ? 2 : 4);
    if (v.wpc <= 0) v.wpc = 2;
    int R = 2, pf = rows <= 4096 ? 1 : 0;
    Fp8Geom g;
    if (tuned && fp8_geom(cols, &g)) {
        const int cu = cu_count();
        /* every round of workgroups but the last is full; the last at least
         * 15/16 full, or the grid is a single round */
        auto grid = [&](int r) { return fp8_plan(g, r, rows, cols, v.wpc, 1).grid; };
        auto full = [&](int r) {
            const int n = grid(r), last = n % cu;
            return n <= cu || last == 0 || last * 16 >= cu * 15;
        };
        if (g.tc == 256) {
            if (sfmt != 0) {
                R = 1;
                pf = 1;
            }
        } else if (rows > 4096) {
            if (!full(2) && full(1)) R = 1;
        } else if (cols >= 4096) {
            if (sfmt == 0 ? full(1) : grid(1) <= cu) {
                R = 1;
                pf = 0;
            } else if (!full(2) && full(4)) {
                R = 4;
                pf = 0;
            }
        }
    }
    R = env_int("DSV4_GPU_FP8_R", R);
    R = R >= 4 ? 4 : R >= 2 ? 2 : 1;
    while (blk_r % R) R >>= 1;                   /* a step stays in one row block */
    v.R = R;
    v.pf = env_int("DSV4_GPU_FP8_PF", pf);
    return v;
}

int fp8_gemv(float *y, const float *x, const uint8_t *W, const void *S, int sfmt,
             int rows, int cols, int blk_r, int blk_c, const Fp8Groups &gp,
             hipStream_t st)
{
    if (rows <= 0 || cols <= 0 || blk_r <= 0 || blk_c <= 0 || gp.n <= 0 || gp.n > 65535) {
        DSV4_ERR("fp8 gemv: bad shape %dx%d blk %dx%d", rows, cols, blk_r, blk_c);
        return -1;
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    Fp8Geom g;
    if (!gp.valu && mx_form(sfmt, cols, blk_r, blk_c)) {
        if (chunked_ok(x, W, "fp8 gemv") != 0) return -1;
        Dsv4Fp8Mx a;
        a.y = y; a.x = x; a.w = W; a.s = (const uint8_t *)S;
        a.rows = rows; a.cols = cols; a.sc = sc; a.blk_r = blk_r; a.blk_c = blk_c;
        a.n = gp.n;
        a.x_stride = gp.x; a.y_stride = gp.y; a.w_stride = gp.w; a.s_stride = gp.s;
        a.list = gp.list;
        for (int i = 0; gp.list && i < gp.n; i++) {
            a.wl[i] = gp.Wl[i]; a.sl[i] = (const uint8_t *)gp.Sl[i];
            a.yl[i] = gp.yl[i]; a.rl[i] = gp.rl[i];
        }
        return dsv4_fp8_mx_launch(a, st);
    }
    if (fp8_geom(cols, &g) && blocking_ok(blk_r, blk_c)) {
        if (chunked_ok(x, W, "fp8 gemv") != 0) return -1;
        /* launch shape (fp8_valu): none of it changes a row's arithmetic */
        const Fp8Valu v = fp8_valu(rows, cols, blk_r, sfmt);
        const int R = v.R, pf = v.pf, wpc = v.wpc;
        if (sfmt == 0) {
            if (pf) launch_gemv_r<0, 1>(g, R, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st);
            else    launch_gemv_r<0, 0>(g, R, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st);
        } else {
            if (pf) launch_gemv_r<1, 1>(g, R, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st);
            else    launch_gemv_r<1, 0>(g, R, y, x, W, S, rows, cols, sc, blk_r, blk_c, wpc, gp, st);
        }
    } else {
        const int grid = (rows + 3) / 4;
        for (int i = 0; i < gp.n; i++) {
            float *yi = y + i * gp.y;
            const float *xi = x + i * gp.x;
            const uint8_t *Wi = W + i * gp.w;
            const void *Si = (const uint8_t *)S + i * gp.s;
            if (sfmt == 0)
                hipLaunchKernelGGL((k_fp8_gemv_generic<0>), dim3(grid), dim3(256), 0, st,
                                   yi, xi, Wi, Si, rows, cols, sc, blk_r, blk_c, 1);
            else
                hipLaunchKernelGGL((k_fp8_gemv_generic<1>), dim3(grid), dim3(256), 0, st,
                                   yi, xi, Wi, Si, rows, cols, sc, blk_r, blk_c, 1);
        }
    }
    HIP_OK(hipGetLastError(), "fp8 gemv launch");
    return 0;
}

/* The attention block's x projections in one launch: its listed FP8
 * matrices (blockIdx.y < gp.n) run k_fp8_gemv's body, its listed BF16
 * matrices the BF16 GEMV's (dsv4_bf16_rows.h); all read the same x. Each
 * part keeps its own launch plan, so every row has the bits of its own
 * GEMV; workgroups past a part's grid leave at once. */
struct XProj {
    const float *x = nullptr;
    int cols = 0;
    Fp8Groups gp;                                  /* FP8: list of gp.n */
    int rows8 = 0, sc = 0, blk_r = 0, blk_c = 0, tc8 = 0, rpw8 = 0, grid8 = 0;
    B16List ls;                                    /* BF16: list of ls.n */
    int tc16 = 0, rpw16 = 0, grid16 = 0;
};

template <int NCH, int R, int SF, int PF, int BNCH, int BR>
__global__ void __launch_bounds__(256)
k_xproj(XProj a)
{
    extern __shared__ float part[];
    const int bx = blockIdx.x, by = blockIdx.y;
    if (by < a.gp.n) {
        if (bx >= a.grid8) return;
        /* (the list supplies each matrix's W, S, y and rows) */
        fp8_rows<NCH, R, SF, PF, 0>(a.gp.yl[0], a.x, a.gp.Wl[0], a.gp.Sl[0], a.rows8, a.cols,
                                    a.sc, a.blk_r, a.blk_c, a.tc8, a.rpw8, a.gp, bx, by, part);
    } else {
        if (bx >= a.grid16) return;
        b16_rows<BNCH, BR>(a.ls.y[0], a.x, a.ls.W[0], a.ls.rows[0], a.cols, a.tc16, a.rpw16,
                           a.ls, bx, by - a.gp.n, part);
    }
}

/* The attention block's q GEMVs and the rest of its prep step in one
 * launch: its listed FP8 matrices (blockIdx.y < gp.n; wq_b and the indexer's
 * wq_b) read qr and normalise their workgroup's copy of it themselves (the
 * prep step's q job, same arithmetic and order: NQ), and the workgroups of
 * row gp.n run the prep step's other jobs (the ring slot's norm and RoPE,
 * the compressor's slot), which nothing in this launch reads. */
struct QProj {
    const float *x = nullptr, *nw = nullptr;
    int cols = 0;
    float eps = 0.0f;
    Fp8Groups gp;
    int rows8 = 0, sc = 0, blk_r = 0, blk_c = 0, tc8 = 0, rpw8 = 0, grid8 = 0;
    Dsv4Prep prep{};
    int nprep = 0;
};

template <int NCH, int R, int SF>
__global__ void __launch_bounds__(256)
k_qproj(QProj a)
{
    extern __shared__ float part[];
    const int bx = blockIdx.x, by = blockIdx.y;
    if (by < a.gp.n) {
        if (bx >= a.grid8) return;
        fp8_rows<NCH, R, SF, 0, 1, 1>(a.gp.yl[0], a.x, a.gp.Wl[0], a.gp.Sl[0], a.rows8, a.cols,
                                      a.sc, a.blk_r, a.blk_c, a.tc8, a.rpw8, a.gp, bx, by, part,
                                      a.nw, a.eps);
    } else {
        if (bx >= a.nprep) return;
        prep_rows(a.prep, bx);
    }
}

} // namespace

int dsv4_fp8_gemv_launch(float *y, const float *x, const uint8_t *W,
                         const void *S, int sfmt, int rows, int cols,
                         int blk_r, int blk_c, hipStream_t st, bool valu)
{
    Fp8Groups gp;
    gp.valu = valu;
    return fp8_gemv(y, x, W, S, sfmt, rows, cols, blk_r, blk_c, gp, st);
}

int dsv4_fp8_gemv_list_launch(const float *x, int cols, int sfmt, int blk_r, int blk_c,
                              int n, const uint8_t *const *W, const void *const *S,
                              float *const *y, const int *rows, hipStream_t st, bool valu)
{
    if (n < 1 || n > FP8_LIST_MAX) {
        DSV4_ERR("fp8 gemv list: %d matrices (1 .. %d)", n, FP8_LIST_MAX);
        return -1;
    }
    Fp8Groups gp;
    gp.n = n;
    gp.list = 1;
    gp.valu = valu;
    int rmax = 0;
    for (int i = 0; i < n; i++) {
        if (rows[i] <= 0 || (((uintptr_t)W[i]) & 15)) {
            DSV4_ERR("fp8 gemv list: matrix %d (%d rows) empty or unaligned", i, rows[i]);
            return -1;
        }
        gp.Wl[i] = W[i]; gp.Sl[i] = S[i]; gp.yl[i] = y[i]; gp.rl[i] = rows[i];
        rmax = rows[i] > rmax ? rows[i] : rmax;
    }
    Fp8Geom g;
    if (!fp8_geom(cols, &g) || !blocking_ok(blk_r, blk_c) || (((uintptr_t)x) & 15)) {
        for (int i = 0; i < n; i++)
            if (dsv4_fp8_gemv_launch(y[i], x, W[i], S[i], sfmt, rows[i], cols, blk_r, blk_c,
                                     st, valu) != 0)
                return -1;
        return 0;
    }
    return fp8_gemv(y[0], x, W[0], S[0], sfmt, rmax, cols, blk_r, blk_c, gp, st);
}

int dsv4_fp8_gemv_groups_launch(float *y, const float *x, const uint8_t *W,
                                const void *S, int sfmt, int rows, int cols, int blk_r,
                                int blk_c, int groups, long long y_stride,
                                long long x_stride, long long w_stride,
                                long long s_stride, hipStream_t st, bool valu)
{
    Fp8Groups gp;
    gp.n = groups;
    gp.valu = valu;
    gp.y = y_stride; gp.x = x_stride; gp.w = w_stride; gp.s = s_stride;
    if (groups > 1 && (((uintptr_t)(x_stride * 4) | (uintptr_t)w_stride) & 15)) {
        DSV4_ERR("fp8 gemv groups: strides break 16-byte alignment");
        return -1;
    }
    return fp8_gemv(y, x, W, S, sfmt, rows, cols, blk_r, blk_c, gp, st);
}

size_t dsv4_fp8_n_scratch_bytes(int rows, int cols, int nt)
{
    return std::max(dsv4_fp8_mxn_scratch_bytes(cols, nt), mfn_scratch_bytes(rows, cols, nt));
}

int dsv4_fp8_gemv_n_launch(float *y, const float *x, const uint8_t *W,
                           const void *S, int sfmt, int rows, int cols,
                           int blk_r, int blk_c, int nt, hipStream_t st, void *xscratch)
{
    if (rows <= 0 || cols <= 0 || nt <= 0 || blk_r <= 0 || blk_c <= 0) {
        DSV4_ERR("fp8 gemv_n: bad shape %dx%d nt %d", rows, cols, nt);
        return -1;
    }
    if (nt == 1)                       /* the GEMV itself: same bits, its launch shape */
        return fp8_gemv(y, x, W, S, sfmt, rows, cols, blk_r, blk_c, Fp8Groups{}, st);
    if (mx_form(sfmt, cols, blk_r, blk_c)) {
        if (chunked_ok(x, W, "fp8 gemv_n") != 0) return -1;
        return dsv4_fp8_mxn_launch(y, x, W, (const uint8_t *)S, rows, cols, blk_r, blk_c, nt,
                                   st, xscratch);
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    Fp8Geom g;
    if (fp8_geom(cols, &g) && blocking_ok(blk_r, blk_c)) {
        if (chunked_ok(x, W, "fp8 gemv_n") != 0) return -1;
        if (sfmt == 0)
            launch_gemv_n<0>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st, xscratch);
        else
            launch_gemv_n<1>(g, y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st, xscratch);
    } else {
        const int grid = (rows + 3) / 4;
        if (sfmt == 0)
            hipLaunchKernelGGL((k_fp8_gemv_generic<0>), dim3(grid), dim3(256), 0, st,
                               y, x, W, S, rows, cols, sc, blk_r, blk_c, nt);
        else
            hipLaunchKernelGGL((k_fp8_gemv_generic<1>), dim3(grid), dim3(256), 0, st,
                               y, x, W, S, rows, cols, sc, blk_r, blk_c, nt);
    }
    HIP_OK(hipGetLastError(), "fp8 gemv_n launch");
    return 0;
}

int dsv4_xproj_launch(const float *x, int cols, int sfmt, int blk_r, int blk_c, int nf,
                      const uint8_t *const *Wf, const void *const *Sf, float *const *yf,
                      const int *rf, int nb, const uint16_t *const *Wb, float *const *yb,
                      const int *rb, hipStream_t st)
{
    auto two = [&]() -> int {
        if (nf > 0 &&
            dsv4_fp8_gemv_list_launch(x, cols, sfmt, blk_r, blk_c, nf, Wf, Sf, yf, rf, st,
                                      true) != 0)
            return -1;
        if (nb > 0 && dsv4_bf16_gemv_list_launch(x, cols, nb, Wb, yb, rb, st) != 0) return -1;
        return 0;
    };
    if (nf < 1 || nb < 1 || nf > FP8_LIST_MAX || nb > B16_LIST_MAX ||
        (sfmt != 0 && sfmt != 1) || env_int("DSV4_GPU_XPROJ", 1) == 0)
        return two();
    Fp8Geom g;
    B16Geom gb;
    bool ok = fp8_geom(cols, &g) && blocking_ok(blk_r, blk_c) && b16_geom(cols, &gb) &&
              (((uintptr_t)x) & 15) == 0;
    int rmf = 0, rmb = 0;
    for (int i = 0; i < nf; i++) {
        ok = ok && rf[i] > 0 && (((uintptr_t)Wf[i]) & 15) == 0;
        rmf = rf[i] > rmf ? rf[i] : rmf;
    }
    for (int i = 0; i < nb; i++) {
        ok = ok && rb[i] > 0 && (((uintptr_t)Wb[i]) & 15) == 0;
        rmb = rb[i] > rmb ? rb[i] : rmb;
    }
    if (!ok) return two();
    const Fp8Valu v = fp8_valu(rmf, cols, blk_r, sfmt, false);
    const Fp8Plan pf = fp8_plan(g, v.R, rmf, cols, v.wpc, nf);
    /* the BF16 part within the FP8 part's grid (DSV4_GPU_XPROJ_CAP=0: its own
     * plan): a wider x grid only adds workgroups of one step each */
    const B16Plan pb = b16_plan(gb, rmb, nb, env_int("DSV4_GPU_XPROJ_CAP", 1) ? pf.grid : 0);
    /* the one combination built: FP8 with 4 chunks per thread, 2 rows per
     * step, prefetch, x in registers; BF16 with 8 chunks per thread, 1 row
     * (hidden 4096 and 7168, the Flash and full shapes) */
    if (g.nch < 4 || v.R != 2 || !v.pf || pf.xl || gb.nch <= 4 || pb.R != 1 || g.wg != 256 ||
        gb.wg != 256)
        return two();
    XProj a;
    a.x = x;
    a.cols = cols;
    a.gp.n = nf;
    a.gp.list = 1;
    a.gp.valu = true;
    for (int i = 0; i < nf; i++) {
        a.gp.Wl[i] = Wf[i]; a.gp.Sl[i] = Sf[i]; a.gp.yl[i] = yf[i]; a.gp.rl[i] = rf[i];
    }
    a.rows8 = rmf; a.sc = (cols + blk_c - 1) / blk_c; a.blk_r = blk_r; a.blk_c = blk_c;
    a.tc8 = g.tc; a.rpw8 = pf.rows_per_wg; a.grid8 = pf.grid;
    a.ls.n = nb;
    for (int i = 0; i < nb; i++) {
        a.ls.W[i] = Wb[i]; a.ls.y[i] = yb[i]; a.ls.rows[i] = rb[i];
    }
    a.tc16 = gb.tc; a.rpw16 = pb.rows_per_wg; a.grid16 = pb.grid;
    const dim3 grid(pf.grid > pb.grid ? pf.grid : pb.grid, nf + nb);
    const size_t lds = pf.lds > pb.lds ? pf.lds : pb.lds;
    if (sfmt == 0)
        hipLaunchKernelGGL((k_xproj<4, 2, 0, 1, 8, 1>), grid, dim3(256), lds, st, a);
    else
        hipLaunchKernelGGL((k_xproj<4, 2, 1, 1, 8, 1>), grid, dim3(256), lds, st, a);
    HIP_OK(hipGetLastError(), "x projections launch");
    return 0;
}

int dsv4_qproj_launch(const float *qr, int cols, const float *nw, float eps, int sfmt,
                      int blk_r, int blk_c, int nf, const uint8_t *const *Wf,
                      const void *const *Sf, float *const *yf, const int *rf,
                      const Dsv4Prep *prep, hipStream_t st)
{
    if (!prep || prep->nj > 1 || nf < 1 || nf > FP8_LIST_MAX) {
        DSV4_ERR("q projections: bad arguments (%d matrices)", nf);
        return -1;
    }
    /* the separate form: the prep step with the q job first, then the list */
    auto two = [&]() -> int {
        Dsv4Prep p = *prep;
        if (p.nj == 1) p.job[1] = p.job[0];
        p.job[0] = Dsv4NormJob{const_cast<float *>(qr), qr, nw, cols, 0};
        p.nj = prep->nj + 1;
        if (dsv4_block_prep_launch(&p, st) != 0) return -1;
        return dsv4_fp8_gemv_list_launch(qr, cols, sfmt, blk_r, blk_c, nf, Wf, Sf, yf, rf, st,
                                         true);
    };
    Fp8Geom g;
    bool ok = env_int("DSV4_GPU_QPROJ", 1) != 0 && (sfmt == 0 || sfmt == 1) && nw &&
              fp8_geom(cols, &g) && blocking_ok(blk_r, blk_c) && (((uintptr_t)qr) & 15) == 0;
    int rm = 0;
    for (int i = 0; i < nf; i++) {
        ok = ok && rf[i] > 0 && (((uintptr_t)Wf[i]) & 15) == 0;
        rm = rf[i] > rm ? rf[i] : rm;
    }
    if (!ok) return two();
    const Fp8Valu v = fp8_valu(rm, cols, blk_r, sfmt, false);
    /* rows per step: 4 (a step stays in one row block), or 2. Four measured
     * faster for the block's q GEMVs (wq_b 32768x1024 and the indexer's
     * 8192x1024 with the prep step: 77.1 -> 74.9 us per CSA step); one row
     * with no prefetch in the x launch measured slower (78.7), so that
     * launch keeps two rows with prefetch. */
    const int qrr = env_int("DSV4_GPU_QPROJ_R", 4) >= 4 && blk_r % 4 == 0 ? 4 : 2;
    const Fp8Plan pf = fp8_plan(g, qrr, rm, cols, v.wpc, nf);
    /* the combinations built: x through LDS (cols <= 2048), 1 or 2 chunks
     * per thread, 2 or 4 rows per step, no prefetch (wq_b's rows), 256
     * threads */
    if (!pf.xl || g.wg != 256 || g.nch > 2 || v.R != 2 || v.pf) return two();
    QProj a;
    a.x = qr; a.nw = nw; a.cols = cols; a.eps = eps;
    a.gp.n = nf; a.gp.list = 1; a.gp.valu = true;
    for (int i = 0; i < nf; i++) {
        a.gp.Wl[i] = Wf[i]; a.gp.Sl[i] = Sf[i]; a.gp.yl[i] = yf[i]; a.gp.rl[i] = rf[i];
    }
    a.rows8 = rm; a.sc = (cols + blk_c - 1) / blk_c; a.blk_r = blk_r; a.blk_c = blk_c;
    a.tc8 = g.tc; a.rpw8 = pf.rows_per_wg; a.grid8 = pf.grid;
    a.prep = *prep;
    a.nprep = prep_wgs(*prep);
    const dim3 grid(pf.grid > a.nprep ? pf.grid : a.nprep, nf + (a.nprep ? 1 : 0));
    static bool opted = false;
    const size_t lds = pf.lds + sizeof(float) * (size_t)cols;   /* + the norm's weights */
    if (!opted) {
        const size_t cap = dsv4_lds_limit();
        const void *fns[] = {(const void *)k_qproj<1, 2, 0>, (const void *)k_qproj<2, 2, 0>,
                             (const void *)k_qproj<1, 2, 1>, (const void *)k_qproj<2, 2, 1>,
                             (const void *)k_qproj<1, 4, 0>, (const void *)k_qproj<2, 4, 0>,
                             (const void *)k_qproj<1, 4, 1>, (const void *)k_qproj<2, 4, 1>};
        for (const void *f : fns) (void)dsv4_lds_optin(f, cap, "q projections");
        opted = true;
    }
#define DSV4_QP(NCH, R, SF) hipLaunchKernelGGL((k_qproj<NCH, R, SF>), grid, dim3(256), lds, st, a)
    if (qrr == 4) {
        if (sfmt == 0) { if (g.nch == 1) DSV4_QP(1, 4, 0); else DSV4_QP(2, 4, 0); }
        else           { if (g.nch == 1) DSV4_QP(1, 4, 1); else DSV4_QP(2, 4, 1); }
    } else {
        if (sfmt == 0) { if (g.nch == 1) DSV4_QP(1, 2, 0); else DSV4_QP(2, 2, 0); }
        else           { if (g.nch == 1) DSV4_QP(1, 2, 1); else DSV4_QP(2, 2, 1); }
    }
#undef DSV4_QP
    HIP_OK(hipGetLastError(), "q projections launch");
    return 0;
}
