/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_bf16_rows.h - the BF16 GEMV's per-workgroup body (dsv4_bf16.hip) as a
 * device function, so that another kernel can run it for some of its
 * workgroups (the attention block's x projections run FP8 and BF16 matrices
 * in one launch, dsv4_fp8.hip). Included inside an anonymous namespace. */
#pragma once

constexpr int B16_PART_MAX = 4096;

/* Several matrices of one width reading the same x in one launch
 * (blockIdx.y = matrix): n == 0 is the plain GEMV. */
constexpr int B16_LIST_MAX = 4;
struct B16List {
    int n = 0;
    const uint16_t *W[B16_LIST_MAX] = {};
    float *y[B16_LIST_MAX] = {};
    int rows[B16_LIST_MAX] = {};
};

struct B16Geom {
    int ch, tc, nch, wg, rg;
};

bool b16_geom(int cols, B16Geom *g)
{
    if (cols <= 0 || (cols & 7)) return false;
    const int ch = cols >> 3;
    int tc, nch;
    if (ch <= 64) {
        tc = 1;
        while (tc < ch) tc <<= 1;
        nch = 1;
    } else {
        tc = 64 * ((ch + 511) / 512);
        if (tc > 256) tc = 256;
        nch = (ch + tc - 1) / tc;
    }
    if (nch > 8) return false;                   /* cols <= 16384 */
    g->ch = ch;
    g->tc = tc;
    g->nch = nch;
    g->wg = tc * (256 / tc);
    g->rg = g->wg / tc;
    return true;
}

/* 8 bf16 (one chunk) dotted with 8 activations, two interleaved chains. */
__device__ __forceinline__ float dot8_bf16(const u32x4 v, const float *xr)
{
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
    float p0 = __uint_as_float(u[0] << 16) * xr[0];
    float p1 = __uint_as_float(u[0] & 0xFFFF0000u) * xr[1];
#pragma unroll
    for (int e = 1; e < 4; e++) {
        p0 = fmaf(__uint_as_float(u[e] << 16), xr[2 * e], p0);
        p1 = fmaf(__uint_as_float(u[e] & 0xFFFF0000u), xr[2 * e + 1], p1);
    }
    return p0 + p1;
}

/* The GEMV of workgroup (bx, by): rows [bx rows_per_wg, +rows_per_wg) of
 * matrix by of the list (or of W). part: LDS of [waves per row][rows_per_wg]
 * floats when a row is wider than one wave. */
template <int NCH, int R>
__device__ __forceinline__ void b16_rows(float *__restrict__ y, const float *__restrict__ x,
                                         const uint16_t *__restrict__ W, int rows, int cols,
                                         int tc, int rows_per_wg, const B16List &ls, int bx,
                                         int by, float *part)
{
    if (ls.n) {
        W = ls.W[by];
        y = ls.y[by];
        rows = ls.rows[by];
        if (bx * rows_per_wg >= rows) return;     /* the whole workgroup */
    }
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = cols >> 3;
    const int lane = tid & 63;
    const int row0 = bx * rows_per_wg;
    const int rend = min(rows, row0 + rows_per_wg);
    const int nloc = rend - row0;
    const uint8_t *Wb = reinterpret_cast<const uint8_t *>(W);
    const size_t rowb = (size_t)cols * 2;

    float xr[NCH][8];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        const int cc = min(c, ch - 1);
        const f32x4 a = ldf4(x + cc * 8), b = ldf4(x + cc * 8 + 4);
        xr[n][0] = a.x; xr[n][1] = a.y; xr[n][2] = a.z; xr[n][3] = a.w;
        xr[n][4] = b.x; xr[n][5] = b.y; xr[n][6] = b.z; xr[n][7] = b.w;
    }

    for (int rb = row0 + g * R; rb < row0 + ((nloc + rg * R - 1) / (rg * R)) * rg * R;
         rb += rg * R) {
        u32x4 v[R][NCH];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = min(rb + i, rend - 1);
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = min(j + n * tc, ch - 1);
                v[i][n] = ldg16_stream(Wb + (size_t)r * rowb + (size_t)c * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            float a = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const float d = a + dot8_bf16(v[i][n], xr[n]);
                a = act[n] ? d : a;
            }
            if (tc <= 64) {
                const float s = seg_sum_rt(a, tc);
                if (j == tc - 1 && rb + i < rend) y[rb + i] = s;
            } else {
                const float s = seg_sum<64>(a);
                const int rl = rb + i - row0;
                if (lane == 63 && rl < nloc) part[(j >> 6) * rows_per_wg + rl] = s;
            }
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


/* Launch plan of the list (or plain) GEMV: R rows per thread per step, the
 * rows each workgroup owns, the grid along x and the dynamic LDS. */
struct B16Plan {
    int R = 1, rows_per_wg = 0, grid = 0;
    size_t lds = 0;
};

inline B16Plan b16_plan(const B16Geom &g, int rows, int nlist, int max_grid = 0)
{
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess ||
            n <= 0)
            n = 256;
        cus = n;
    }
    B16Plan p;
    /* two rows per thread per step while the loads fit the registers */
    p.R = g.nch <= 4 ? 2 : 1;
    const int step_rows = g.rg * p.R;
    const int nm = nlist ? nlist : 1;
    const int want = (2 * cus + nm - 1) / nm;       /* two workgroups per CU */
    const int wpr = g.tc > 64 ? g.tc / 64 : 1;
    int spw = ((rows + step_rows - 1) / step_rows + want - 1) / want;
    /* at most max_grid workgroups along x (a launch that shares its grid) */
    if (max_grid > 0) {
        const int nsteps = (rows + step_rows - 1) / step_rows;
        const int spw_min = (nsteps + max_grid - 1) / max_grid;
        if (spw < spw_min) spw = spw_min;
    }
    const int max_spw = B16_PART_MAX / wpr / step_rows;
    if (spw > max_spw) spw = max_spw;
    if (spw < 1) spw = 1;
    p.rows_per_wg = spw * step_rows;
    p.grid = (rows + p.rows_per_wg - 1) / p.rows_per_wg;
    p.lds = g.tc > 64 ? sizeof(float) * (size_t)wpr * p.rows_per_wg : 0;
    return p;
}
