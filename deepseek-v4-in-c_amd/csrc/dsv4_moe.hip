/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe.hip - fused MXFP4 routed-expert matvec on gfx950.
 *
 * Computes the routed half of the reference's moe() for one token
 * (src/model/dsv4_layer.c:380, :412-476): for each selected expert k,
 *     acc_k = w2_k . swiglu(w1_k . x, w3_k . x)          (expert_forward :199)
 * and then out[i] = sum_k w[k] * acc_k[i], strictly in k order (:471-475).
 * The packed format is the reference's: E2M1 nibbles, low nibble = even
 * element, one E8M0 scale per 1x32 block (dsv4_quant.h:141-164,
 * dsv4_matmul.c:320-345); SwiGLU is dsv4_swiglu (dsv4_ops.c:60-78).
 *
 * THREE PASSES, all bandwidth-bound streams of the experts' bytes:
 *   A  gate/up: each "h-row" (k, o) reads w1_k row o and w3_k row o together
 *      (2 x hidden/2 bytes + 2 x hidden/32 scale bytes), reduces both dots and
 *      applies SwiGLU in registers; h[k][o] goes to a small scratch (topk x
 *      inter floats).
 *   B  down: each (k, i) reads w2_k row i (inter/2 bytes) against h[k];
 *      acc[k][i] to scratch (topk x hidden floats).
 *   C  combine: out[i] = ((0 + w0*acc0[i]) + w1*acc1[i]) + ... in k order,
 *      each multiply and add rounded separately (this file is built with
 *      -ffp-contract=off).
 *   Row geometry follows the FP8 GEMV: a 16-byte chunk is 32 elements = one
 *   scale block; a row is split over TC threads with NCH chunks each, x slice
 *   in VGPRs, R rows in flight per thread, fixed DPP reduction tree.
 *
 * Expert pointers come from a device table indexed by expert id, and the ids
 * and router weights are read from device memory, so routing computed on the
 * device needs no host round trip. An id that is out of range or not resident
 * yields NaN outputs (never a wild read).
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

namespace {

struct Fp4Geom { int ch, tc, nch, wg, rg; };

/* ch = 16-byte chunks per row = elements / 32. */
bool fp4_geom(int elems, Fp4Geom *g)
{
    if (elems <= 0 || (elems & 31)) return false;
    const int ch = elems >> 5;
    int tc, nch;
    if (ch <= 64) {
        tc = 1;
        while (tc < ch) tc <<= 1;
        nch = 1;
    } else {
        tc = 64 * ((ch + 127) / 128);
        nch = (ch + tc - 1) / tc;
    }
    if (tc > 256 || nch > 2) return false;     /* rows <= 16384 elements */
    g->ch = ch; g->tc = tc; g->nch = nch;
    g->wg = tc * (256 / tc);
    g->rg = g->wg / tc;
    return true;
}

/* 32 E2M1 elements (one 16-byte chunk) dotted with 32 activations. */
__device__ __forceinline__ float dot32(const u32x4 v, const float *xr)
{
    float w[32];
    dec_fp4x8(v.x, w + 0);
    dec_fp4x8(v.y, w + 8);
    dec_fp4x8(v.z, w + 16);
    dec_fp4x8(v.w, w + 24);
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

__device__ __forceinline__ void load_x32(float *xr, const float *x, bool ok)
{
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const f32x4 v = ok ? ldf4(x + q * 4) : f32x4{0, 0, 0, 0};
        xr[q * 4 + 0] = v.x; xr[q * 4 + 1] = v.y;
        xr[q * 4 + 2] = v.z; xr[q * 4 + 3] = v.w;
    }
}

/* dsv4_swiglu for one element (dsv4_ops.c:60-78): up clamped to [-L, L],
 * gate clamped above only, silu(g) = g / (1 + expf(-g)). */
__device__ __forceinline__ float swiglu1(float g, float u, float limit)
{
    if (limit > 0.0f) {
        if (u > limit) u = limit;
        if (u < -limit) u = -limit;
        if (g > limit) g = limit;
        const float s = g / (1.0f + expf(-g));
        return s * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

__device__ __forceinline__ const Dsv4ExpertDev *
expert_of(const Dsv4ExpertDev *table, int n_table, const int *idx, int k)
{
    const int e = idx[k];
    if (e < 0 || e >= n_table) return nullptr;
    const Dsv4ExpertDev *p = table + e;
    return p->w1 ? p : nullptr;
}

/* Pass A. h-row hr = k*inter + o. */
template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_moe_gate_up(float *__restrict__ h, const float *__restrict__ x,
              const Dsv4ExpertDev *__restrict__ table, int n_table,
              const int *__restrict__ idx, int topk, int hidden, int inter,
              float limit, int tc, int tiles_per_wg, int ntiles)
{
    __shared__ float red[4][2 * R];
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = hidden >> 5;
    const int wid = tid >> 6, lane = tid & 63;
    const int hrows = topk * inter;
    const size_t rowb = (size_t)hidden / 2, rows_s = (size_t)ch;

    float xr[NCH][32];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        load_x32(xr[n], x + c * 32, act[n]);
    }

    const int t0 = blockIdx.x * tiles_per_wg;
    const int t1 = min(ntiles, t0 + tiles_per_wg);
    for (int tile = t0; tile < t1; ++tile) {
        const int hbase = (tile * rg + g) * R;
        u32x4 wg_[R][NCH], wu_[R][NCH];
        float sg[R][NCH], su[R][NCH];
        bool bad[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int hr = hbase + i;
            const bool ok = hr < hrows;
            const int k = ok ? hr / inter : 0;
            const int o = ok ? hr - k * inter : 0;
            const Dsv4ExpertDev *e = ok ? expert_of(table, n_table, idx, k) : nullptr;
            bad[i] = ok && !e;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = j + n * tc;
                if (e && act[n]) {
                    wg_[i][n] = ld16_stream(e->w1 + (size_t)o * rowb + (size_t)c * 16);
                    wu_[i][n] = ld16_stream(e->w3 + (size_t)o * rowb + (size_t)c * 16);
                    sg[i][n] = dec_e8m0(e->s1[(size_t)o * rows_s + c]);
                    su[i][n] = dec_e8m0(e->s3[(size_t)o * rows_s + c]);
                } else {
                    wg_[i][n] = u32x4{0, 0, 0, 0};
                    wu_[i][n] = u32x4{0, 0, 0, 0};
                    sg[i][n] = 0.0f;
                    su[i][n] = 0.0f;
                }
            }
        }
        float ag[R], au[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                a = fmaf(dot32(wg_[i][n], xr[n]), sg[i][n], a);
                b = fmaf(dot32(wu_[i][n], xr[n]), su[i][n], b);
            }
            ag[i] = a; au[i] = b;
        }
        if (tc <= 64) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float gs = seg_sum_rt(ag[i], tc);
                const float us = seg_sum_rt(au[i], tc);
                const int hr = hbase + i;
                if (j == tc - 1 && hr < hrows)
                    h[hr] = bad[i] ? __builtin_nanf("") : swiglu1(gs, us, limit);
            }
        } else {
            const int wpr = tc >> 6;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float gs = seg_sum<64>(ag[i]);
                const float us = seg_sum<64>(au[i]);
                if (lane == 63) { red[wid][2 * i] = gs; red[wid][2 * i + 1] = us; }
            }
            __syncthreads();
            if (tid < rg * R) {
                const int gg = tid / R, ii = tid - gg * R;
                const int hr = (tile * rg + gg) * R + ii;
                float gs = red[gg * wpr][2 * ii], us = red[gg * wpr][2 * ii + 1];
                for (int w = 1; w < wpr; w++) {
                    gs += red[gg * wpr + w][2 * ii];
                    us += red[gg * wpr + w][2 * ii + 1];
                }
                if (hr < hrows) {
                    const int k = hr / inter;
                    const bool b = !expert_of(table, n_table, idx, k);
                    h[hr] = b ? __builtin_nanf("") : swiglu1(gs, us, limit);
                }
            }
            __syncthreads();
        }
    }
}

/* Pass B. Row dr = k*hidden + i; x = h[k]. */
template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_moe_down(float *__restrict__ acc, const float *__restrict__ h,
           const Dsv4ExpertDev *__restrict__ table, int n_table,
           const int *__restrict__ idx, int topk, int hidden, int inter,
           int tc, int tiles_per_wg, int ntiles, int tiles_per_expert)
{
    __shared__ float red[4][R];
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = inter >> 5;
    const int wid = tid >> 6, lane = tid & 63;
    const size_t rowb = (size_t)inter / 2, rows_s = (size_t)ch;

    float xr[NCH][32];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) act[n] = j + n * tc < ch;
    int cur_k = -1;
    const Dsv4ExpertDev *e = nullptr;

    const int t0 = blockIdx.x * tiles_per_wg;
    const int t1 = min(ntiles, t0 + tiles_per_wg);
    for (int tile = t0; tile < t1; ++tile) {
        const int k = tile / tiles_per_expert;
        const int tt = tile - k * tiles_per_expert;
        if (k != cur_k) {
            cur_k = k;
            e = expert_of(table, n_table, idx, k);
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = j + n * tc;
                load_x32(xr[n], h + (size_t)k * inter + c * 32, act[n]);
            }
        }
        const int ibase = (tt * rg + g) * R;
        u32x4 wv[R][NCH];
        float sv[R][NCH];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = ibase + i;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = j + n * tc;
                if (e && act[n] && r < hidden) {
                    wv[i][n] = ld16_stream(e->w2 + (size_t)r * rowb + (size_t)c * 16);
                    sv[i][n] = dec_e8m0(e->s2[(size_t)r * rows_s + c]);
                } else {
                    wv[i][n] = u32x4{0, 0, 0, 0};
                    sv[i][n] = 0.0f;
                }
            }
        }
        float a[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            float s = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) s = fmaf(dot32(wv[i][n], xr[n]), sv[i][n], s);
            a[i] = s;
        }
        const float nanv = __builtin_nanf("");
        if (tc <= 64) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = seg_sum_rt(a[i], tc);
                const int r = ibase + i;
                if (j == tc - 1 && r < hidden)
                    acc[(size_t)k * hidden + r] = e ? v : nanv;
            }
        } else {
            const int wpr = tc >> 6;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float v = seg_sum<64>(a[i]);
                if (lane == 63) red[wid][i] = v;
            }
            __syncthreads();
            if (tid < rg * R) {
                const int gg = tid / R, ii = tid - gg * R;
                const int r = (tt * rg + gg) * R + ii;
                float s = red[gg * wpr][ii];
                for (int w = 1; w < wpr; w++) s += red[gg * wpr + w][ii];
                if (r < hidden) acc[(size_t)k * hidden + r] = e ? s : nanv;
            }
            __syncthreads();
        }
    }
}

/* Pass C: dsv4_layer.c:471-475, in k order, no fused multiply-add. */
__global__ void __launch_bounds__(256)
k_moe_combine(float *__restrict__ out, const float *__restrict__ acc,
              const float *__restrict__ w, int topk, int hidden)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    float o = 0.0f;
    for (int k = 0; k < topk; k++) {
        const float p = w[k] * acc[(size_t)k * hidden + i];
        o = o + p;
    }
    out[i] = o;
}

template <int NCH, int R>
void launch_a(const Fp4Geom &g, float *h, const float *x,
              const Dsv4ExpertDev *table, int n_table, const int *idx,
              int topk, int hidden, int inter, float limit, hipStream_t st)
{
    const int per = g.rg * R;
    const int hrows = topk * inter;
    const int ntiles = (hrows + per - 1) / per;
    const int want = ntiles < 2048 ? ntiles : 2048;
    const int tpw = (ntiles + want - 1) / want;
    const int grid = (ntiles + tpw - 1) / tpw;
    hipLaunchKernelGGL((k_moe_gate_up<NCH, R>), dim3(grid), dim3(g.wg), 0, st,
                       h, x, table, n_table, idx, topk, hidden, inter, limit,
                       g.tc, tpw, ntiles);
}

template <int NCH, int R>
void launch_b(const Fp4Geom &g, float *acc, const float *h,
              const Dsv4ExpertDev *table, int n_table, const int *idx,
              int topk, int hidden, int inter, hipStream_t st)
{
    const int per = g.rg * R;
    const int tpe = (hidden + per - 1) / per;
    const int ntiles = tpe * topk;
    const int want = ntiles < 2048 ? ntiles : 2048;
    const int tpw = (ntiles + want - 1) / want;
    const int grid = (ntiles + tpw - 1) / tpw;
    hipLaunchKernelGGL((k_moe_down<NCH, R>), dim3(grid), dim3(g.wg), 0, st,
                       acc, h, table, n_table, idx, topk, hidden, inter, g.tc,
                       tpw, ntiles, tpe);
}

int pick_r(int rows, int rg)
{
    for (int cand = 4; cand >= 2; cand >>= 1)
        if ((rows + rg * cand - 1) / (rg * cand) >= 2048) return cand;
    return 1;
}

} // namespace

int dsv4_moe_fp4_launch(float *d_out, const float *d_x,
                        const Dsv4ExpertDev *d_table, int n_table,
                        const int *d_idx, const float *d_w, int topk,
                        int hidden, int inter, float limit, float *hbuf,
                        float *accbuf, hipStream_t st)
{
    Fp4Geom ga, gb;
    if (topk <= 0 || !fp4_geom(hidden, &ga) || !fp4_geom(inter, &gb)) {
        DSV4_ERR("moe: unsupported shape hidden %d inter %d topk %d "
                 "(need multiples of 32, at most 16384)", hidden, inter, topk);
        return -1;
    }
    const int ra = pick_r(topk * inter, ga.rg);
    if (ga.nch == 1) {
        if (ra == 4) launch_a<1, 4>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
        else if (ra == 2) launch_a<1, 2>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
        else launch_a<1, 1>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
    } else {
        if (ra == 4) launch_a<2, 4>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
        else if (ra == 2) launch_a<2, 2>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
        else launch_a<2, 1>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, st);
    }
    HIP_OK(hipGetLastError(), "moe gate/up launch");
    const int rb = pick_r(topk * hidden, gb.rg);
    if (gb.nch == 1) {
        if (rb == 4) launch_b<1, 4>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
        else if (rb == 2) launch_b<1, 2>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
        else launch_b<1, 1>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
    } else {
        if (rb == 4) launch_b<2, 4>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
        else if (rb == 2) launch_b<2, 2>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
        else launch_b<2, 1>(gb, accbuf, hbuf, d_table, n_table, d_idx, topk, hidden, inter, st);
    }
    HIP_OK(hipGetLastError(), "moe down launch");
    hipLaunchKernelGGL(k_moe_combine, dim3((hidden + 255) / 256), dim3(256), 0,
                       st, d_out, accbuf, d_w, topk, hidden);
    HIP_OK(hipGetLastError(), "moe combine launch");
    return 0;
}
