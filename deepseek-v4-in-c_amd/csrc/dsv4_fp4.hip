/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_fp4.hip - MXFP4 GEMV for resident FP4 matrices on gfx950.
 *
 * What it computes is dsv4_matmul_fp4 (reference src/core/dsv4_matmul.c:
 * 320-345): W is e2m1 nibbles, row o stored in cols/2 bytes (element i in the
 * low nibble of byte i/2 when i is even, the high one when odd,
 * dsv4_quant.h:155-164), with one E8M0 scale per (blk_r x blk_c) block,
 *   y[o] = sum over blk_c-column blocks of (block dot) * e8m0(S[(o/blk_r)*sc +
 *          c0/blk_c]).
 * It is how dsv4_gpu_mmq runs an FP4 matrix made resident by dsv4_gpu_upload
 * -- the routed and shared experts of the reference's expert_forward
 * (dsv4_layer.c:199-206), one matrix per call. The fused routed-expert pass
 * (dsv4_moe_mx.hip) is the batch-1 decode path; this one serves the
 * reference's own dispatch (dsv4_mmq, dsv4_matmul.c:525-546).
 *
 * APPROACH (bandwidth-bound, one 16-byte chunk = 32 elements = one 32-column
 * scale block or a part of a wider one):
 *   - The workgroup stages x into LDS once (cols floats); every wave then
 *     reads its 32-float slices from there.
 *   - A wave owns one row at a time, R rows per step with all their chunks'
 *     loads issued before any arithmetic; lane l takes chunks l, l+64, ...
 *     so each wave instruction moves 1 KiB of one row.
 *   - Decode is v_cvt_scalef32_pk_f32_fp4 (exact), a 32-element dot in four
 *     fp32 chains, then one FMA with the chunk's block scale. The lane
 *     partials meet in the fixed DPP tree of seg_sum.
 * NUMERICS: fp32 (the reference accumulates the block dot and the row total
 * in double); within 1e-5 vector-scaled relative of it.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <stdlib.h>

namespace {

constexpr int F4_WAVES = 4;
constexpr int F4_MAXCOLS = 16384;

/* 32 decoded elements of one chunk dotted with 32 activations from LDS. */
__device__ __forceinline__ float f4_dot32(const u32x4 v, const float *xs)
{
    float w[32];
    dec_fp4x8(v.x, w + 0);
    dec_fp4x8(v.y, w + 8);
    dec_fp4x8(v.z, w + 16);
    dec_fp4x8(v.w, w + 24);
    float xr[32];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const f32x4 t = *reinterpret_cast<const f32x4 *>(xs + 4 * q);
        xr[4 * q + 0] = t.x; xr[4 * q + 1] = t.y;
        xr[4 * q + 2] = t.z; xr[4 * q + 3] = t.w;
    }
    float p0 = w[0] * xr[0], p1 = w[1] * xr[1];
    float p2 = w[2] * xr[2], p3 = w[3] * xr[3];
#pragma unroll
    for (int e = 4; e < 32; e += 4) {
        p0 = fmaf(w[e + 0], xr[e + 0], p0);
        p1 = fmaf(w[e + 1], xr[e + 1], p1);
        p2 = fmaf(w[e + 2], xr[e + 2], p2);
        p3 = fmaf(w[e + 3], xr[e + 3], p3);
    }
    return (p0 + p1) + (p2 + p3);
}

/* Workgroup: rows [row0, row0 + rows_per_wg), R rows per wave per step; NCH
 * chunks per lane (64 * NCH >= cols / 32). Every load is issued
 * unconditionally -- chunks past the row end reload the last chunk and rows
 * past the range the last row, their results discarded -- so no branch sits
 * between a load and the wait that counts it. */
template <int NCH, int R>
__global__ void __launch_bounds__(F4_WAVES * 64)
k_fp4_gemv(float *__restrict__ y, const float *__restrict__ x,
           const uint8_t *__restrict__ W, const uint8_t *__restrict__ S, int rows,
           int cols, int sc, int blk_r, int blk_c, int rows_per_wg)
{
    extern __shared__ __attribute__((aligned(16))) float xs[];   /* [cols] */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ch = cols >> 5;                                    /* chunks per row */
    const size_t rowb = (size_t)cols >> 1;
    for (int i = tid; i < (cols >> 2); i += blockDim.x)
        *reinterpret_cast<f32x4 *>(xs + 4 * i) = ldf4(x + 4 * i);
    __syncthreads();

    int cb[NCH];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = lane + 64 * n;
        act[n] = c < ch;
        cb[n] = (min(c, ch - 1) * 32) / blk_c;
    }
    const int row0 = blockIdx.x * rows_per_wg;
    const int rend = min(rows, row0 + rows_per_wg);
    for (int rb = row0 + w * R; rb < rend; rb += F4_WAVES * R) {
        u32x4 v[R][NCH];
        uint32_t sv[R][NCH];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = min(rb + i, rend - 1);
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = min(lane + 64 * n, ch - 1);
                v[i][n] = ldg16_stream(W + (size_t)r * rowb + (size_t)c * 16);
                sv[i][n] = ldg8(S + (size_t)(r / blk_r) * sc + cb[n]);
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            float acc = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = min(lane + 64 * n, ch - 1);
                const float d = fmaf(f4_dot32(v[i][n], xs + c * 32), dec_e8m0(sv[i][n]), acc);
                acc = act[n] ? d : acc;
                /* one chunk's decode at a time: interleaving them would only
                 * hold more registers (the loads are all in flight already) */
                __builtin_amdgcn_sched_barrier(0);
            }
            acc = seg_sum<64>(acc);
            if (lane == 63 && rb + i < rend) y[rb + i] = acc;
        }
    }
}

template <int NCH>
void f4_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S, int rows,
               int cols, int sc, int blk_r, int blk_c, hipStream_t st)
{
    /* two rows per step in flight while they fit the registers */
    constexpr int R = NCH >= 4 ? 1 : 2;
    static bool opted = false;                  /* x of up to 64 KB in LDS */
    if (!opted) {
        (void)dsv4_lds_optin((const void *)k_fp4_gemv<NCH, R>, F4_MAXCOLS * sizeof(float),
                             "fp4 gemv");
        opted = true;
    }
    /* 4 rows per workgroup (one per wave): at expert shapes the grid's
     * parallelism matters more than staging x once per more rows (cold, us,
     * 16 / 8 / 4 rows: 2048x7168 10.1 / 6.8 / 6.3, 7168x2048 6.6 / 6.5 /
     * 6.2, 1024x4096 7.2 / 5.0 / 4.5, 4096x4096 7.6 / 7.1 / 7.1). A wave
     * owns whole rows, so the split changes no row's arithmetic.
     * DSV4_GPU_FP4_RPW overrides it. */
    const char *e = getenv("DSV4_GPU_FP4_RPW");
    const int rows_per_wg = e && atoi(e) > 0 ? atoi(e) : 4;
    const int grid = (rows + rows_per_wg - 1) / rows_per_wg;
    hipLaunchKernelGGL((k_fp4_gemv<NCH, R>), dim3(grid), dim3(F4_WAVES * 64),
                       (size_t)cols * sizeof(float), st, y, x, W, S, rows, cols, sc,
                       blk_r, blk_c, rows_per_wg);
}

/* Batched (prefill): y[t][rows] for x[t][cols], t < nt, each (row, token)
 * with k_fp4_gemv's arithmetic -- the same chunk dots, scale FMAs in chunk
 * order and DPP tree -- so every token's row is bit-identical to the
 * single-token GEMV. A wave holds its R rows' chunks and scale bytes in
 * VGPRs and runs every token over them: the weights leave HBM once per batch
 * (the reference's one pass per batch, dsv4_matmul_fp4_n at
 * dsv4_matmul.c:378-428 and dsv4_mmq_n :560-591). The tokens' x pass through
 * LDS in blocks of tbx (a block is staged once per workgroup when nt <= tbx,
 * else once per row step). */
template <int NCH, int R>
__global__ void __launch_bounds__(F4_WAVES * 64)
k_fp4_gemv_n(float *__restrict__ y, const float *__restrict__ x,
             const uint8_t *__restrict__ W, const uint8_t *__restrict__ S, int rows,
             int cols, int sc, int blk_r, int blk_c, int nt, int tbx)
{
    extern __shared__ __attribute__((aligned(16))) float xs[];   /* [tbx][cols] */
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ch = cols >> 5;
    const size_t rowb = (size_t)cols >> 1;
    const int nq = cols >> 2;                                    /* f32x4 per token */
    int cb[NCH];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = lane + 64 * n;
        act[n] = c < ch;
        cb[n] = (min(c, ch - 1) * 32) / blk_c;
    }
    const int rb = blockIdx.x * (F4_WAVES * R) + w * R;          /* this wave's rows */
    u32x4 v[R][NCH];
    uint32_t sv[R][NCH];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int r = min(rb + i, rows - 1);
#pragma unroll
        for (int n = 0; n < NCH; n++) {
            const int c = min(lane + 64 * n, ch - 1);
            v[i][n] = ldg16_stream(W + (size_t)r * rowb + (size_t)c * 16);
            sv[i][n] = ldg8(S + (size_t)(r / blk_r) * sc + cb[n]);
        }
    }
    for (int t0 = 0; t0 < nt; t0 += tbx) {
        const int tb = min(tbx, nt - t0);
        __syncthreads();                         /* the previous block's reads */
        for (int i = tid; i < tb * nq; i += blockDim.x)
            *reinterpret_cast<f32x4 *>(xs + 4 * i) = ldf4(x + (size_t)t0 * cols + 4 * i);
        __syncthreads();
        for (int t = 0; t < tb; t++) {
            const float *xt = xs + (size_t)t * cols;
#pragma unroll
            for (int i = 0; i < R; i++) {
                float acc = 0.0f;
#pragma unroll
                for (int n = 0; n < NCH; n++) {
                    const int c = min(lane + 64 * n, ch - 1);
                    const float d = fmaf(f4_dot32(v[i][n], xt + c * 32), dec_e8m0(sv[i][n]),
                                         acc);
                    acc = act[n] ? d : acc;
                }
                acc = seg_sum<64>(acc);
                if (lane == 63 && rb + i < rows) y[(size_t)(t0 + t) * rows + rb + i] = acc;
            }
        }
    }
}

template <int NCH>
void f4n_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S, int rows,
                int cols, int sc, int blk_r, int blk_c, int nt, hipStream_t st)
{
    constexpr int R = NCH >= 4 ? 1 : 2;
    static bool opted = false;                  /* up to 64 KB of x in LDS */
    if (!opted) {
        (void)dsv4_lds_optin((const void *)k_fp4_gemv_n<NCH, R>, F4_MAXCOLS * sizeof(float),
                             "fp4 gemv_n");
        opted = true;
    }
    int tbx = F4_MAXCOLS / cols;                /* tokens per LDS block */
    if (tbx > 8) tbx = 8;
    if (tbx > nt) tbx = nt;
    const int grid = (rows + F4_WAVES * R - 1) / (F4_WAVES * R);
    hipLaunchKernelGGL((k_fp4_gemv_n<NCH, R>), dim3(grid), dim3(F4_WAVES * 64),
                       (size_t)tbx * cols * sizeof(float), st, y, x, W, S, rows, cols, sc,
                       blk_r, blk_c, nt, tbx);
}

} // namespace

int dsv4_fp4_gemv_n_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S,
                           int rows, int cols, int blk_r, int blk_c, int nt, hipStream_t st)
{
    if (nt == 1) return dsv4_fp4_gemv_launch(y, x, W, S, rows, cols, blk_r, blk_c, st);
    if (nt < 1 || !dsv4_fp4_gemv_ok(rows, cols, blk_r, blk_c) ||
        (((uintptr_t)x | (uintptr_t)W) & 15)) {
        DSV4_ERR("fp4 gemv_n: unsupported shape %dx%d blk %dx%d, %d tokens, or unaligned "
                 "operands", rows, cols, blk_r, blk_c, nt);
        return -1;
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    const int ch = cols >> 5;
    if (ch <= 64)       f4n_launch<1>(y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st);
    else if (ch <= 128) f4n_launch<2>(y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st);
    else if (ch <= 256) f4n_launch<4>(y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st);
    else                f4n_launch<8>(y, x, W, S, rows, cols, sc, blk_r, blk_c, nt, st);
    HIP_OK(hipGetLastError(), "fp4 gemv_n launch");
    return 0;
}

bool dsv4_fp4_gemv_ok(int rows, int cols, int blk_r, int blk_c)
{
    return rows > 0 && cols > 0 && cols <= F4_MAXCOLS && (cols & 31) == 0 &&
           blk_r >= 1 && blk_c >= 32 && (blk_c & 31) == 0;
}

int dsv4_fp4_gemv_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S,
                         int rows, int cols, int blk_r, int blk_c, hipStream_t st)
{
    if (!dsv4_fp4_gemv_ok(rows, cols, blk_r, blk_c) ||
        (((uintptr_t)x | (uintptr_t)W) & 15)) {
        DSV4_ERR("fp4 gemv: unsupported shape %dx%d blk %dx%d or unaligned operands",
                 rows, cols, blk_r, blk_c);
        return -1;
    }
    const int sc = (cols + blk_c - 1) / blk_c;
    const int ch = cols >> 5;
    if (ch <= 64)       f4_launch<1>(y, x, W, S, rows, cols, sc, blk_r, blk_c, st);
    else if (ch <= 128) f4_launch<2>(y, x, W, S, rows, cols, sc, blk_r, blk_c, st);
    else if (ch <= 256) f4_launch<4>(y, x, W, S, rows, cols, sc, blk_r, blk_c, st);
    else                f4_launch<8>(y, x, W, S, rows, cols, sc, blk_r, blk_c, st);
    HIP_OK(hipGetLastError(), "fp4 gemv launch");
    return 0;
}
