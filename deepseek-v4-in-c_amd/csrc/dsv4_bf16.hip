/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_bf16.hip - BF16 GEMV for resident BF16 matrices on gfx950.
 *
 * What it computes is dsv4_matmul_bf16 (reference src/core/dsv4_matmul.c:
 * 275-291): y[o] = (float) sum_i bf16(W[o][i]) * x[i]. It is how
 * dsv4_gpu_mmq runs a BF16 matrix made resident by dsv4_gpu_upload -- the
 * router gate of moe() (dsv4_layer.c:374) and the LM head
 * (dsv4_run.c:467-474) go through the reference's dsv4_mmq dispatch
 * (dsv4_matmul.c:525-546) like every other matrix.
 *
 * APPROACH (bandwidth-bound, one multiply-add per 2 weight bytes)
 *   - A row is split over TC threads (a power of two up to 64, or a multiple
 *     of 64 up to 256); thread j owns the 16-byte chunks (8 elements) j,
 *     j+TC, ... of every row it visits (NCH <= 8 of them, so rows up to
 *     16384 columns). Consecutive lanes read consecutive chunks: one wave
 *     instruction moves 1 KiB of one row.
 *   - The thread's slice of x (NCH x 8 floats) is loaded once into VGPRs and
 *     reused for every row; workgroups are persistent over a contiguous
 *     range of rows.
 *   - A thread works on R rows at once, all R*NCH loads in flight before any
 *     arithmetic, issued unconditionally (rows past the end reload the last
 *     row, chunks past the row end the last chunk; their results are
 *     discarded).
 *   - bf16 -> f32 is exact (a shift); 8 f32 FMAs per chunk in two chains.
 *     Lane partials meet in the fixed DPP tree, and across the waves of a
 *     row in wave order through LDS.
 * NUMERICS: fp32 (the reference accumulates in double); within 1e-5
 * vector-scaled relative of it. TC, NCH and the trees depend on cols only,
 * so a row's bits do not depend on R or the grid.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

namespace {

#include "dsv4_bf16_rows.h"

template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_bf16_gemv(float *__restrict__ y, const float *__restrict__ x,
            const uint16_t *__restrict__ W, int rows, int cols, int tc, int rows_per_wg,
            B16List ls)
{
    extern __shared__ float part[];                 /* [waves per row][rows_per_wg] */
    b16_rows<NCH, R>(y, x, W, rows, cols, tc, rows_per_wg, ls, (int)blockIdx.x,
                     (int)blockIdx.y, part);
}

/* Batched (prefill): y[t][rows] for x[t][cols], t < nt, each (row, token)
 * with k_bf16_gemv's arithmetic -- the same thread geometry, chunk chains,
 * DPP tree and wave order -- so every token's row is bit-identical to the
 * single-token GEMV. A row group holds its R rows' chunks in VGPRs and runs
 * every token over them: the weights leave HBM once per batch (dsv4_mmq_n,
 * dsv4_matmul.c:560-591). The tokens' x pass through LDS in blocks of tbx;
 * each row's per-wave partials (rows wider than one wave) meet in LDS in
 * wave order. */
template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_bf16_gemv_n(float *__restrict__ y, const float *__restrict__ x,
              const uint16_t *__restrict__ W, int rows, int cols, int tc, int nt, int tbx)
{
    extern __shared__ __attribute__((aligned(16))) float xsn[];   /* [tbx][cols], red */
    float *red = xsn + (size_t)tbx * cols;                        /* [4 waves][R][tbx] */
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = cols >> 3;
    const int lane = tid & 63, wid = tid >> 6;
    const int nq = cols >> 2;
    const uint8_t *Wb = reinterpret_cast<const uint8_t *>(W);
    const size_t rowb = (size_t)cols * 2;
    const int rb = blockIdx.x * rg * R + g * R;                  /* this group's rows */
    bool act[NCH];
    u32x4 v[R][NCH];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int r = min(rb + i, rows - 1);
#pragma unroll
        for (int n = 0; n < NCH; n++) {
            const int c = j + n * tc;
            act[n] = c < ch;
            v[i][n] = ldg16_stream(Wb + (size_t)r * rowb + (size_t)min(c, ch - 1) * 16);
        }
    }
    for (int t0 = 0; t0 < nt; t0 += tbx) {
        const int tb = min(tbx, nt - t0);
        __syncthreads();                         /* the previous block's reads */
        for (int i = tid; i < tb * nq; i += blockDim.x)
            *reinterpret_cast<f32x4 *>(xsn + 4 * i) = ldf4(x + (size_t)t0 * cols + 4 * i);
        __syncthreads();
        for (int t = 0; t < tb; t++) {
            const float *xt = xsn + (size_t)t * cols;
            float xr[NCH][8];
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int cc = min(j + n * tc, ch - 1);
                const f32x4 a = *reinterpret_cast<const f32x4 *>(xt + cc * 8);
                const f32x4 b = *reinterpret_cast<const f32x4 *>(xt + cc * 8 + 4);
                xr[n][0] = a.x; xr[n][1] = a.y; xr[n][2] = a.z; xr[n][3] = a.w;
                xr[n][4] = b.x; xr[n][5] = b.y; xr[n][6] = b.z; xr[n][7] = b.w;
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
                    if (j == tc - 1 && rb + i < rows) y[(size_t)(t0 + t) * rows + rb + i] = s;
                } else {
                    const float s = seg_sum<64>(a);
                    if (lane == 63) red[(wid * R + i) * tbx + t] = s;
                }
            }
        }
        if (tc > 64) {
            __syncthreads();
            const int wpr = tc >> 6;
            for (int q = tid; q < rg * R * tb; q += blockDim.x) {
                const int gg = q / (R * tb), rem = q - gg * R * tb;
                const int i = rem / tb, tt = rem - i * tb;
                const int rr = blockIdx.x * rg * R + gg * R + i;
                float s = red[((gg * wpr) * R + i) * tbx + tt];
                for (int ww = 1; ww < wpr; ww++) s += red[((gg * wpr + ww) * R + i) * tbx + tt];
                if (rr < rows) y[(size_t)(t0 + tt) * rows + rr] = s;
            }
        }
    }
}

template <int NCH>
void b16n_launch(const B16Geom &g, float *y, const float *x, const uint16_t *W, int rows,
                 int cols, int nt, hipStream_t st)
{
    constexpr int R = NCH <= 4 ? 4 : 2;
    static bool opted = false;                  /* up to 64 KB of x in LDS */
    if (!opted) {
        (void)dsv4_lds_optin((const void *)k_bf16_gemv_n<NCH, R>,
                             16384 * sizeof(float) + 4 * R * 8 * sizeof(float), "bf16 gemv_n");
        opted = true;
    }
    int tbx = 16384 / cols;                     /* tokens per LDS block */
    if (tbx > 8) tbx = 8;
    if (tbx > nt) tbx = nt;
    const int per = g.rg * R;                   /* rows per workgroup */
    const int grid = (rows + per - 1) / per;
    const size_t lds = sizeof(float) * ((size_t)tbx * cols + 4 * R * tbx);
    hipLaunchKernelGGL((k_bf16_gemv_n<NCH, R>), dim3(grid), dim3(g.wg), lds, st, y, x, W,
                       rows, cols, g.tc, nt, tbx);
}

template <int NCH>
void b16_launch(const B16Geom &g, float *y, const float *x, const uint16_t *W, int rows,
                int cols, const B16List &ls, hipStream_t st)
{
    /* the plan's R: two rows per thread per step for up to 4 chunks */
    constexpr int R = NCH <= 4 ? 2 : 1;
    const B16Plan p = b16_plan(g, rows, ls.n);
    const int nm = ls.n ? ls.n : 1;
    hipLaunchKernelGGL((k_bf16_gemv<NCH, R>), dim3(p.grid, nm), dim3(g.wg), p.lds, st, y, x, W,
                       rows, cols, g.tc, p.rows_per_wg, ls);
}

int b16_dispatch(const B16Geom &g, float *y, const float *x, const uint16_t *W, int rows,
                 int cols, const B16List &ls, hipStream_t st)
{
    switch (g.nch) {
    case 1: b16_launch<1>(g, y, x, W, rows, cols, ls, st); break;
    case 2: b16_launch<2>(g, y, x, W, rows, cols, ls, st); break;
    case 3: case 4: b16_launch<4>(g, y, x, W, rows, cols, ls, st); break;
    default: b16_launch<8>(g, y, x, W, rows, cols, ls, st); break;
    }
    HIP_OK(hipGetLastError(), "bf16 gemv launch");
    return 0;
}

} // namespace

bool dsv4_bf16_gemv_ok(int rows, int cols)
{
    B16Geom g;
    return rows > 0 && b16_geom(cols, &g);
}

int dsv4_bf16_gemv_launch(float *y, const float *x, const uint16_t *W, int rows, int cols,
                          hipStream_t st)
{
    B16Geom g;
    if (rows <= 0 || !b16_geom(cols, &g) || (((uintptr_t)x | (uintptr_t)W) & 15)) {
        DSV4_ERR("bf16 gemv: unsupported shape %dx%d or unaligned operands", rows, cols);
        return -1;
    }
    return b16_dispatch(g, y, x, W, rows, cols, B16List{}, st);
}

int dsv4_bf16_gemv_n_launch(float *y, const float *x, const uint16_t *W, int rows, int cols,
                            int nt, hipStream_t st)
{
    if (nt == 1) return dsv4_bf16_gemv_launch(y, x, W, rows, cols, st);
    B16Geom g;
    if (nt < 1 || rows <= 0 || !b16_geom(cols, &g) || (((uintptr_t)x | (uintptr_t)W) & 15)) {
        DSV4_ERR("bf16 gemv_n: unsupported shape %dx%d, %d tokens, or unaligned operands",
                 rows, cols, nt);
        return -1;
    }
    switch (g.nch) {
    case 1: b16n_launch<1>(g, y, x, W, rows, cols, nt, st); break;
    case 2: b16n_launch<2>(g, y, x, W, rows, cols, nt, st); break;
    case 3: case 4: b16n_launch<4>(g, y, x, W, rows, cols, nt, st); break;
    default: b16n_launch<8>(g, y, x, W, rows, cols, nt, st); break;
    }
    HIP_OK(hipGetLastError(), "bf16 gemv_n launch");
    return 0;
}

int dsv4_bf16_gemv_list_launch(const float *x, int cols, int n, const uint16_t *const *W,
                               float *const *y, const int *rows, hipStream_t st)
{
    B16Geom g;
    if (n < 1 || n > B16_LIST_MAX || !b16_geom(cols, &g) || (((uintptr_t)x) & 15)) {
        DSV4_ERR("bf16 gemv list: %d matrices of width %d not supported", n, cols);
        return -1;
    }
    B16List ls;
    ls.n = n;
    int rmax = 0;
    for (int i = 0; i < n; i++) {
        if (rows[i] <= 0 || (((uintptr_t)W[i]) & 15)) {
            DSV4_ERR("bf16 gemv list: matrix %d (%d rows) empty or unaligned", i, rows[i]);
            return -1;
        }
        ls.W[i] = W[i]; ls.y[i] = y[i]; ls.rows[i] = rows[i];
        rmax = rows[i] > rmax ? rows[i] : rmax;
    }
    return b16_dispatch(g, y[0], x, W[0], rmax, cols, ls, st);
}
