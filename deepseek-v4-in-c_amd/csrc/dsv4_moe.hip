/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_moe.hip - fused MXFP4 routed-expert matvec on gfx950, VALU form.
 *
 * This is the general path, for any hidden / inter that are multiples of 32:
 * it decodes the nibbles with v_cvt_scalef32_pk_f32_fp4 and accumulates with
 * fp32 FMAs. Shapes that are multiples of 128 take the matrix-core form in
 * dsv4_moe_mx.hip instead, which the launcher there selects.
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

#include <stdlib.h>

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


__device__ __forceinline__ const Dsv4ExpertDev *
expert_of(const Dsv4ExpertDev *table, int n_table, const int *idx, int k)
{
    const int e = idx[k];
    if (e < 0 || e >= n_table) return nullptr;
    const Dsv4ExpertDev *p = table + e;
    return p->w1 ? p : nullptr;
}

/* The selected experts' tensors, resolved once per workgroup into LDS (the
 * id lookup and the table read are two dependent loads that would otherwise
 * sit in front of every weight load). A missing expert has w1 == nullptr. */
constexpr int MOE_KMAX = 64;

__device__ __forceinline__ void resolve_experts(Dsv4ExpertDev *sx,
                                                const Dsv4ExpertDev *table,
                                                int n_table, const int *idx,
                                                int topk)
{
    const int t = threadIdx.x;
    if (t < topk) {
        const Dsv4ExpertDev *e = expert_of(table, n_table, idx, t);
        if (e) sx[t] = *e;
        else   sx[t] = Dsv4ExpertDev{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    }
    __syncthreads();
}

/* Pass A. h-row hr = k*inter + o. A workgroup owns the contiguous h-rows
 * [row0, row0 + rows_per_wg) and walks them in steps of rg*R; rows wider
 * than one wave leave per-wave gate/up partials in LDS, summed in wave order
 * after one barrier, then SwiGLU. */
template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_moe_gate_up(float *__restrict__ h, const float *__restrict__ x,
              const Dsv4ExpertDev *__restrict__ table, int n_table,
              const int *__restrict__ idx, int topk, int hidden, int inter,
              float limit, int tc, int rows_per_wg)
{
    extern __shared__ float part[];          /* [2][waves per row][rows_per_wg] */
    __shared__ Dsv4ExpertDev sx[MOE_KMAX];
    resolve_experts(sx, table, n_table, idx, topk);
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = hidden >> 5;
    const int lane = tid & 63;
    const int hrows = topk * inter;
    const size_t rowb = (size_t)hidden / 2, rows_s = (size_t)ch;
    const int row0 = blockIdx.x * rows_per_wg;
    const int rend = min(hrows, row0 + rows_per_wg);
    const int nloc = rend - row0;
    const int step_rows = rg * R;
    const int nsteps = (nloc + step_rows - 1) / step_rows;
    const int wpr = tc > 64 ? tc >> 6 : 1;

    float xr[NCH][32];
    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) {
        const int c = j + n * tc;
        act[n] = c < ch;
        load_x32(xr[n], x + c * 32, act[n]);
    }

    u32x4 wg_[R][NCH], wu_[R][NCH];
    uint32_t sg_[R][NCH], su_[R][NCH];
    bool bad[R];

    /* This row group's first h-row as (expert slot, row): advanced by
     * step_rows per step without a division. Rows past the workgroup's end
     * read row rend-1 and are not stored; a missing expert reads x (valid
     * memory) and stores NaN. Every load is unconditional, so no branch
     * stands between the loads and the waits that count them. */
    const int hr0 = row0 + g * R;
    int kq = hr0 / inter, oq = hr0 - kq * inter;
    const int klast = (rend - 1) / inter, olast = (rend - 1) - klast * inter;
    const uint8_t *xb = (const uint8_t *)x;
    int cc[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) cc[n] = min(j + n * tc, ch - 1);

    auto load = [&](int hr, int k_, int o_, u32x4 (*G)[NCH], u32x4 (*U)[NCH],
                    uint32_t (*SG)[NCH], uint32_t (*SU)[NCH], bool *B) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            int ki = k_, oi = o_ + i;
            if (oi >= inter) { oi -= inter; ki++; }
            const bool ok = hr + i < rend;
            if (!ok) { ki = klast; oi = olast; }
            const Dsv4ExpertDev &e = sx[ki];
            const bool miss = e.w1 == nullptr;
            const uint8_t *p1 = miss ? xb : e.w1 + (size_t)oi * rowb;
            const uint8_t *p3 = miss ? xb : e.w3 + (size_t)oi * rowb;
            const uint8_t *q1 = miss ? xb : e.s1 + (size_t)oi * rows_s;
            const uint8_t *q3 = miss ? xb : e.s3 + (size_t)oi * rows_s;
            B[i] = ok && miss;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                G[i][n] = ldg16_stream(p1 + (size_t)cc[n] * 16);
                U[i][n] = ldg16_stream(p3 + (size_t)cc[n] * 16);
                SG[i][n] = ldg8(q1 + cc[n]);
                SU[i][n] = ldg8(q3 + cc[n]);
            }
        }
    };
    auto advance = [&](int &k_, int &o_) {
        o_ += step_rows;
        while (o_ >= inter) { o_ -= inter; k_++; }
    };

    if (nsteps > 0) load(hr0, kq, oq, wg_, wu_, sg_, su_, bad);
    for (int step = 0; step < nsteps; ++step) {
        const int rbase = row0 + step * step_rows + g * R;
        int kn = kq, on = oq;
        advance(kn, on);

        float ag[R], au[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const float da = fmaf(dot32(wg_[i][n], xr[n]), dec_e8m0(sg_[i][n]), a);
                const float db = fmaf(dot32(wu_[i][n], xr[n]), dec_e8m0(su_[i][n]), b);
                a = act[n] ? da : a;
                b = act[n] ? db : b;
            }
            ag[i] = a; au[i] = b;
        }
        if (tc <= 64) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float gs = seg_sum_rt(ag[i], tc);
                const float us = seg_sum_rt(au[i], tc);
                const int hr = rbase + i;
                if (j == tc - 1 && hr < rend)
                    h[hr] = bad[i] ? __builtin_nanf("") : swiglu1(gs, us, limit);
            }
        } else {
            const int w = j >> 6;
#pragma unroll
            for (int i = 0; i < R; i++) {
                const float gs = seg_sum<64>(ag[i]);
                const float us = seg_sum<64>(au[i]);
                const int rl = rbase + i - row0;
                if (lane == 63 && rl < nloc) {
                    part[(0 * wpr + w) * rows_per_wg + rl] = gs;
                    part[(1 * wpr + w) * rows_per_wg + rl] = us;
                }
            }
        }
        /* the next step's loads go out once this step's weights are consumed
         * (a register double buffer measured no faster: the other resident
         * workgroups keep the memory queues full) */
        if (step + 1 < nsteps) load(rbase + step_rows, kn, on, wg_, wu_, sg_, su_, bad);
        kq = kn;
        oq = on;
    }

    if (tc > 64) {
        __syncthreads();
        for (int rl = tid; rl < nloc; rl += blockDim.x) {
            float gs = part[rl], us = part[wpr * rows_per_wg + rl];
            for (int w = 1; w < wpr; w++) {
                gs += part[w * rows_per_wg + rl];
                us += part[(wpr + w) * rows_per_wg + rl];
            }
            const int hr = row0 + rl;
            const int k = hr / inter;
            h[hr] = sx[k].w1 ? swiglu1(gs, us, limit) : __builtin_nanf("");
        }
    }
}

/* Pass B + C. A workgroup owns the output rows [row0, row0 + rg*R) (one
 * step); it walks the experts in k order with the next expert's weights and
 * h slice in flight while the current one is reduced, keeping acc_k in LDS;
 * then out[i] = ((0 + w0*acc0) + w1*acc1) + ... in k order, each multiply
 * and add rounded separately (dsv4_layer.c:471-475). */
template <int NCH, int R>
__global__ void __launch_bounds__(256)
k_moe_down(float *__restrict__ out, const float *__restrict__ h,
           const Dsv4ExpertDev *__restrict__ table, int n_table,
           const int *__restrict__ idx, const float *__restrict__ wts,
           int topk, int hidden, int inter, int tc)
{
    extern __shared__ float accl[];          /* [topk][waves per row][rows_per_wg] */
    __shared__ Dsv4ExpertDev sx[MOE_KMAX];
    resolve_experts(sx, table, n_table, idx, topk);
    const int tid = threadIdx.x;
    const int g = tid / tc, j = tid - g * tc;
    const int rg = blockDim.x / tc;
    const int ch = inter >> 5;
    const int lane = tid & 63;
    const size_t rowb = (size_t)inter / 2, rows_s = (size_t)ch;
    const int rows_per_wg = rg * R;
    const int row0 = blockIdx.x * rows_per_wg;
    const int rend = min(hidden, row0 + rows_per_wg);
    const int nloc = rend - row0;
    const int rbase = row0 + g * R;
    const int wpr = tc > 64 ? tc >> 6 : 1;
    const float nanv = __builtin_nanf("");

    bool act[NCH];
#pragma unroll
    for (int n = 0; n < NCH; n++) act[n] = j + n * tc < ch;

    float xr[NCH][32], nx[NCH][32];
    u32x4 wv[R][NCH], nw[R][NCH];
    uint32_t sv[R][NCH], ns[R][NCH];

    auto load = [&](int k, float (*X)[32], u32x4 (*Wv)[NCH], uint32_t (*Sv)[NCH]) {
        const Dsv4ExpertDev *e = sx[k].w1 ? &sx[k] : nullptr;
#pragma unroll
        for (int n = 0; n < NCH; n++)
            load_x32(X[n], h + (size_t)k * inter + (j + n * tc) * 32, act[n]);
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int r = rbase + i;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = j + n * tc;
                if (e && act[n] && r < rend) {
                    Wv[i][n] = ldg16_stream(e->w2 + (size_t)r * rowb + (size_t)c * 16);
                    Sv[i][n] = ldg8(e->s2 + (size_t)r * rows_s + c);
                } else {
                    Wv[i][n] = u32x4{0, 0, 0, 0};
                    Sv[i][n] = 0u;
                }
            }
        }
    };

    load(0, xr, wv, sv);
    for (int k = 0; k < topk; k++) {
        if (k + 1 < topk) load(k + 1, nx, nw, ns);
        const bool ek = sx[k].w1 != nullptr;
#pragma unroll
        for (int i = 0; i < R; i++) {
            float a = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++)
                a = fmaf(dot32(wv[i][n], xr[n]), dec_e8m0(sv[i][n]), a);
            const int rl = rbase + i - row0;
            if (tc <= 64) {
                const float v = seg_sum_rt(a, tc);
                if (j == tc - 1 && rl < nloc)
                    accl[(size_t)k * rows_per_wg + rl] = ek ? v : nanv;
            } else {
                const float v = seg_sum<64>(a);
                if (lane == 63 && rl < nloc)
                    accl[((size_t)k * wpr + (j >> 6)) * rows_per_wg + rl] = ek ? v : nanv;
            }
        }
#pragma unroll
        for (int n = 0; n < NCH; n++)
#pragma unroll
            for (int q = 0; q < 32; q++) xr[n][q] = nx[n][q];
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int n = 0; n < NCH; n++) { wv[i][n] = nw[i][n]; sv[i][n] = ns[i][n]; }
    }
    __syncthreads();
    for (int rl = tid; rl < nloc; rl += blockDim.x) {
        float o = 0.0f;
        for (int k = 0; k < topk; k++) {
            float a = accl[((size_t)k * wpr) * rows_per_wg + rl];
            for (int w = 1; w < wpr; w++) a += accl[((size_t)k * wpr + w) * rows_per_wg + rl];
            const float p = wts[k] * a;
            o = o + p;
        }
        out[row0 + rl] = o;
    }
}

/* Pass B + combine, wave per expert slot. A workgroup owns the output rows
 * [r0, r0 + RB); wave w takes slots k = w, w + nwaves, ...: its 32*NCH
 * elements of h_k stay in VGPRs, it requests all RB rows of w2_k (one 1 KB
 * contiguous load per row and chunk) before reducing any of them, and each
 * row's dot lands in LDS. Then out[i] = ((0 + w0*acc0[i]) + w1*acc1[i]) + ...
 * in k order, each multiply and add rounded separately (dsv4_layer.c:
 * 471-475). */
template <int NCH, int RB>
__global__ void __launch_bounds__(512)
k_moe_down_w(float *__restrict__ out, const float *__restrict__ h,
             const Dsv4ExpertDev *__restrict__ table, int n_table,
             const int *__restrict__ idx, const float *__restrict__ wts,
             int topk, int hidden, int inter)
{
    __shared__ float accl[MOE_KMAX][RB];
    const int r0 = blockIdx.x * RB;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int ch = inter >> 5;
    const size_t rowb = (size_t)inter / 2, rows_s = (size_t)ch;

    for (int k = w; k < topk; k += nw) {
        const int e = idx[k];
        const Dsv4ExpertDev E = (e >= 0 && e < n_table)
            ? table[e] : Dsv4ExpertDev{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        if (!E.w1) {
            for (int i = lane; i < RB; i += 64) accl[k][i] = __builtin_nanf("");
            continue;
        }
        bool act[NCH];
#pragma unroll
        for (int n = 0; n < NCH; n++) act[n] = lane + 64 * n < ch;
        u32x4 wv[RB][NCH];
        uint32_t sv[RB][NCH];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const int r = r0 + i;
#pragma unroll
            for (int n = 0; n < NCH; n++) {
                const int c = lane + 64 * n;
                const bool ok = act[n] && r < hidden;
                wv[i][n] = ok ? ldg16_stream(E.w2 + (size_t)r * rowb + (size_t)c * 16)
                              : u32x4{0, 0, 0, 0};
                sv[i][n] = ok ? ldg8(E.s2 + (size_t)r * rows_s + c) : 0u;
            }
        }
        float xr[NCH][32];
#pragma unroll
        for (int n = 0; n < NCH; n++)
            load_x32(xr[n], h + (size_t)k * inter + (lane + 64 * n) * 32, act[n]);
#pragma unroll
        for (int i = 0; i < RB; i++) {
            float a = 0.0f;
#pragma unroll
            for (int n = 0; n < NCH; n++)
                a = fmaf(dot32(wv[i][n], xr[n]), dec_e8m0(sv[i][n]), a);
            const float v = seg_sum<64>(a);
            if (lane == 63) accl[k][i] = v;
        }
    }
    __syncthreads();
    const int nloc = min(RB, hidden - r0);
    for (int i = threadIdx.x; i < nloc; i += blockDim.x) {
        float o = 0.0f;
        for (int kk = 0; kk < topk; kk++) {
            const float p = wts[kk] * accl[kk][i];
            o = o + p;
        }
        out[r0 + i] = o;
    }
}

int g_moe_cus = 0;

int moe_env(const char *name, int dflt)
{
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}

int moe_cus()
{
    if (!g_moe_cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        g_moe_cus = n;
    }
    return g_moe_cus;
}

/* Rows per workgroup: about `wpc` workgroups per CU over `rows` rows walked
 * in steps of `step`, capped so the per-row LDS fits. */
int rows_per_wg_for(int rows, int step, int wpc, size_t lds_per_row, size_t lds_cap)
{
    const int nsteps = (rows + step - 1) / step;
    const int want = wpc * moe_cus();
    int spw = (nsteps + want - 1) / want;
    if (spw < 1) spw = 1;
    if (lds_per_row) {
        const int max_rows = (int)(lds_cap / lds_per_row);
        const int max_spw = max_rows / step;
        if (max_spw < 1) return -1;
        if (spw > max_spw) spw = max_spw;
    }
    return spw * step;
}

template <int NCH, int R>
int launch_a(const Fp4Geom &g, float *h, const float *x,
             const Dsv4ExpertDev *table, int n_table, const int *idx,
             int topk, int hidden, int inter, float limit, int wpc,
             hipStream_t st)
{
    const int hrows = topk * inter;
    const int wpr = g.tc > 64 ? g.tc / 64 : 1;
    const size_t per_row = g.tc > 64 ? 2 * sizeof(float) * wpr : 0;
    const int rpw = rows_per_wg_for(hrows, g.rg * R, wpc, per_row, 32 * 1024);
    if (rpw <= 0) return -1;
    const int grid = (hrows + rpw - 1) / rpw;
    hipLaunchKernelGGL((k_moe_gate_up<NCH, R>), dim3(grid), dim3(g.wg),
                       per_row * rpw, st, h, x, table, n_table, idx, topk, hidden,
                       inter, limit, g.tc, rpw);
    return 0;
}

template <int NCH, int R>
int launch_b(const Fp4Geom &g, float *out, const float *h,
             const Dsv4ExpertDev *table, int n_table, const int *idx,
             const float *w, int topk, int hidden, int inter, hipStream_t st)
{
    const int wpr = g.tc > 64 ? g.tc / 64 : 1;
    const int rpw = g.rg * R;
    const size_t lds = sizeof(float) * (size_t)topk * wpr * rpw;
    const int grid = (hidden + rpw - 1) / rpw;
    hipLaunchKernelGGL((k_moe_down<NCH, R>), dim3(grid), dim3(g.wg), lds, st, out,
                       h, table, n_table, idx, w, topk, hidden, inter, g.tc);
    return 0;
}

} // namespace

int dsv4_moe_fp4_valu_launch(float *d_out, const float *d_x,
                             const Dsv4ExpertDev *d_table, int n_table,
                             const int *d_idx, const float *d_w, int topk,
                             int hidden, int inter, float limit, float *hbuf,
                             hipStream_t st)
{
    Fp4Geom ga, gb;
    if (topk <= 0 || topk > MOE_KMAX || !fp4_geom(hidden, &ga) || !fp4_geom(inter, &gb)) {
        DSV4_ERR("moe: unsupported shape hidden %d inter %d topk %d "
                 "(need multiples of 32, at most 16384, topk <= 64)", hidden, inter, topk);
        return -1;
    }
    /* Launch shape (no effect on the arithmetic of a row), from a sweep at
     * the C3 shape: two rows per thread, no prefetch, two workgroups per CU
     * for the gate/up pass; two rows per thread for the row-group down pass. */
    constexpr int wa = 2;
    int rc = ga.nch == 1
                 ? launch_a<1, 2>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, wa, st)
                 : launch_a<2, 2>(ga, hbuf, d_x, d_table, n_table, d_idx, topk, hidden, inter, limit, wa, st);
    if (rc != 0) { DSV4_ERR("moe: gate/up shape does not fit"); return -1; }
    HIP_OK(hipGetLastError(), "moe gate/up launch");
    if (inter <= 4096 && moe_env("DSV4_GPU_MOE_DOWNW", 1)) {
        const int nw = topk < 8 ? topk : 8;
        const int rbw = moe_env("DSV4_GPU_MOE_RBW", 32) >= 32 ? 32 : 16;
        if (inter <= 2048 && rbw == 32)
            hipLaunchKernelGGL((k_moe_down_w<1, 32>), dim3((hidden + 31) / 32), dim3(64 * nw),
                               0, st, d_out, hbuf, d_table, n_table, d_idx, d_w, topk,
                               hidden, inter);
        else if (inter <= 2048)
            hipLaunchKernelGGL((k_moe_down_w<1, 16>), dim3((hidden + 15) / 16), dim3(64 * nw),
                               0, st, d_out, hbuf, d_table, n_table, d_idx, d_w, topk,
                               hidden, inter);
        else
            hipLaunchKernelGGL((k_moe_down_w<2, 8>), dim3((hidden + 7) / 8), dim3(64 * nw),
                               0, st, d_out, hbuf, d_table, n_table, d_idx, d_w, topk,
                               hidden, inter);
        rc = 0;
    } else if (gb.nch == 1) {
        rc = launch_b<1, 2>(gb, d_out, hbuf, d_table, n_table, d_idx, d_w, topk, hidden, inter, st);
    } else {
        rc = launch_b<2, 2>(gb, d_out, hbuf, d_table, n_table, d_idx, d_w, topk, hidden, inter, st);
    }
    if (rc != 0) { DSV4_ERR("moe: down shape does not fit"); return -1; }
    HIP_OK(hipGetLastError(), "moe down launch");
    return 0;
}
