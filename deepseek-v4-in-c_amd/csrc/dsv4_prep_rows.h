/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_prep_rows.h - the attention block's norms (weighted RMSNorm with an
 * optional RoPE tail) and its prep step's per-workgroup body (dsv4_attnblk.hip)
 * as device functions, so that another launch can run them for some of its
 * workgroups (the block's q GEMVs, dsv4_fp8.hip). Included inside an
 * anonymous namespace. */
#pragma once

constexpr int NR_THREADS = 256;

/* The workgroup's total of v, in a fixed order, in every thread. */
__device__ __forceinline__ double block_sum_d(double v)
{
    __shared__ double part[NR_THREADS / 64];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = part[0];
#pragma unroll
    for (int w = 1; w < NR_THREADS / 64; w++) t += part[w];
    return t;
}

/* Vector b = blockIdx.x: y = src_b (times inv = 1/sqrt(mean square + eps)
 * when norm, then times w when given), its last rd elements rotated at pos.
 * Every element is read and written by one thread (the pairs of the tail by
 * the thread that owns the pair), so dst may alias src. Up to NR_E elements
 * per thread every load (x, w, the pair's cos / sin) is issued at the start,
 * before the norm's reduction, so the kernel waits for memory once. */
constexpr int NR_E = 4;

__device__ __forceinline__ void
norm_rope_vec(float *y, const float *x, const float *__restrict__ w, int n, int norm, float eps,
              int rd, const float *__restrict__ cs, const float *__restrict__ sn, int pos,
              int half, int inverse)
{
    const int tid = threadIdx.x;
    const int t0 = n - rd;
    if (n <= NR_E * NR_THREADS && rd / 2 <= NR_THREADS) {
        float xv[NR_E], wv[NR_E];
#pragma unroll
        for (int e = 0; e < NR_E; e++) {
            const int i = tid + e * NR_THREADS;
            xv[e] = i < n ? x[i] : 0.0f;
            wv[e] = (w && i < t0) ? w[i] : 1.0f;
        }
        /* this thread's RoPE pair */
        const int pp = tid;
        const bool hp = pp < rd / 2;
        float re = 0.0f, im = 0.0f, wa = 1.0f, wb = 1.0f, c = 1.0f, s0 = 0.0f;
        if (hp) {
            re = x[t0 + 2 * pp];
            im = x[t0 + 2 * pp + 1];
            if (w) { wa = w[t0 + 2 * pp]; wb = w[t0 + 2 * pp + 1]; }
            c = cs[(size_t)pos * half + pp];
            s0 = sn[(size_t)pos * half + pp];
        }
        float inv = 1.0f;
        if (norm) {
            double sq = 0.0;
#pragma unroll
            for (int e = 0; e < NR_E; e++) {
                const double v = (double)xv[e];
                sq += v * v;
            }
            sq = block_sum_d(sq);
            inv = (float)(1.0 / sqrt(sq / (double)n + (double)eps));
        }
#pragma unroll
        for (int e = 0; e < NR_E; e++) {
            const int i = tid + e * NR_THREADS;
            if (i < t0) {
                float v = xv[e];
                if (norm) v = v * inv;
                if (w) v = wv[e] * v;
                y[i] = v;
            }
        }
        if (hp) {
            if (norm) { re = re * inv; im = im * inv; }
            if (w) { re = wa * re; im = wb * im; }
            const float sv = inverse ? -s0 : s0;
            y[t0 + 2 * pp] = re * c - im * sv;
            y[t0 + 2 * pp + 1] = re * sv + im * c;
        }
        return;
    }
    float inv = 1.0f;
    if (norm) {
        double sq = 0.0;
        for (int i = tid; i < n; i += NR_THREADS) {
            const double v = (double)x[i];
            sq += v * v;
        }
        sq = block_sum_d(sq);
        inv = (float)(1.0 / sqrt(sq / (double)n + (double)eps));
    }
    for (int i = tid; i < t0; i += NR_THREADS) {
        float v = x[i];
        if (norm) v = v * inv;
        if (w) v = w[i] * v;
        y[i] = v;
    }
    for (int p = tid; p < rd / 2; p += NR_THREADS) {
        const int i = t0 + 2 * p;
        float re = x[i], im = x[i + 1];
        if (norm) { re = re * inv; im = im * inv; }
        if (w) { re = w[i] * re; im = w[i + 1] * im; }
        const float c = cs[(size_t)pos * half + p];
        const float s0 = sn[(size_t)pos * half + p];
        const float s = inverse ? -s0 : s0;
        y[i] = re * c - im * s;
        y[i + 1] = re * s + im * c;
    }
}

/* Workgroup bx of the prep step: norm job bx (bx < nj), else its slice of
 * the compressor's slot update. */
__device__ __forceinline__ void prep_rows(const Dsv4Prep &a, int bx)
{
    if (bx < a.nj) {
        const Dsv4NormJob &j = a.job[bx];
        norm_rope_vec(j.dst, j.src, j.w, j.n, 1, a.eps, j.rd, a.cs, a.sn, a.pos, a.half, 0);
        return;
    }
    const int c = (bx - a.nj) * NR_THREADS + threadIdx.x;
    if (c >= a.width) return;
    a.kvs[c] = a.kv_in[c];
    a.scs[c] = a.sc_in[c] + a.apr[c];
}

/* The workgroups of a prep step. */
inline int prep_wgs(const Dsv4Prep &a)
{
    return a.nj + (a.width + NR_THREADS - 1) / NR_THREADS;
}
