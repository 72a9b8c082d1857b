/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_attnblk.hip - the small kernels of the attention block on gfx950.
 *
 * attention() (reference src/model/dsv4_layer.c:213-336) runs, for one token:
 * five to nine GEMVs (the FP8 / BF16 kernels of this library), the CSA
 * score / top-k / sparse attention (dsv4_mla.hip), and the element-wise steps
 * here:
 *   - k_norm_rope: RMSNorm (dsv4_ops.c:24-31, weighted) or the per-head norm
 *     of q (dsv4_layer.c:223-229, unweighted), then RoPE of the last rd
 *     elements (dsv4_rope.c:105-119, interleaved pairs; inverse negates the
 *     sine) -- either step optional, one workgroup per vector, the result
 *     written where the caller wants it (a ring slot of the KV cache, a
 *     compressed row);
 *   - k_comp_update / k_comp_pool: the compressor's decode step
 *     (dsv4_compress.c:77-137): the token into its slot with score + ape,
 *     and when a window closes the per-channel softmax pool over the slots
 *     (ratio 4: the previous window's first halves and the current window's
 *     second halves), then the ratio-4 slide;
 *   - k_attn_idxs: the row list of the sparse attention -- the window's ring
 *     slots newest first (dsv4_attn.c:118-128), then the compressed rows
 *     (all of them, or the indexer's selection) offset past the window
 *     (dsv4_indexer.c:113-117).
 *
 * NUMERICS. Sums of squares and the pool's sums are in double like the
 * reference's, but as trees over the workgroup instead of one sequential
 * chain; the float inverse 1/sqrt(...) they feed rounds away the difference
 * (the double sums agree to about n * 2^-53). Every float multiply and add is
 * the reference's, in its order (-ffp-contract=off). expf is the device's.
 * The pool's channel loop is sequential over slots exactly as the
 * reference's.
 */
#include "dsv4_dev.h"
#include "dsv4_internal.h"

#include <math.h>

namespace {

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

__global__ void __launch_bounds__(NR_THREADS)
k_norm_rope(float *dst, int dst_stride, const float *src, int src_stride,
            const float *__restrict__ w, int n, int norm, float eps, int rd,
            const float *__restrict__ cs, const float *__restrict__ sn, int pos, int half,
            int inverse)
{
    const float *x = src + (size_t)blockIdx.x * src_stride;
    float *y = dst + (size_t)blockIdx.x * dst_stride;
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

/* The token's slot: kv_state row = kv_in, score_state row = score_in + ape
 * row (the caller passes the slot's and the phase's rows). */
__global__ void __launch_bounds__(NR_THREADS)
k_comp_update(float *__restrict__ kvs, float *__restrict__ scs,
              const float *__restrict__ kv_in, const float *__restrict__ sc_in,
              const float *__restrict__ apr, int width)
{
    const int c = blockIdx.x * NR_THREADS + threadIdx.x;
    if (c >= width) return;
    kvs[c] = kv_in[c];
    scs[c] = sc_in[c] + apr[c];
}

/* Channel c of the closing window's pool. ov (ratio 4): slots 0..ratio-1
 * are the previous window's first halves (columns c), slots ratio..2ratio-1
 * the current window's second halves (columns hd + c); afterwards the
 * current window slides into the previous one. A thread touches only the
 * columns c and hd + c, so the slide needs no barrier. */
__global__ void __launch_bounds__(NR_THREADS)
k_comp_pool(float *__restrict__ out, float *__restrict__ kvst, float *__restrict__ scst,
            int ratio, int hd, int ov)
{
    const int c = blockIdx.x * NR_THREADS + threadIdx.x;
    if (c >= hd) return;
    const int width = ov ? 2 * hd : hd;
    const int slots = ov ? 2 * ratio : ratio;
    float mx = -INFINITY;
    for (int s = 0; s < slots; s++) {
        const int col = (ov && s >= ratio) ? hd + c : c;
        const float v = scst[(size_t)s * width + col];
        if (v > mx) mx = v;
    }
    float r = 0.0f;
    if (mx != -INFINITY) {
        double den = 0.0, acc = 0.0;
        for (int s = 0; s < slots; s++) {
            const int col = (ov && s >= ratio) ? hd + c : c;
            const float v = scst[(size_t)s * width + col];
            if (v == -INFINITY) continue;
            const double e = (double)expf(v - mx);
            den += e;
            acc += e * (double)kvst[(size_t)s * width + col];
        }
        r = (float)(acc / den);
    }
    out[c] = r;
    if (ov) {
        for (int s = 0; s < ratio; s++) {
            const size_t to = (size_t)s * width, from = (size_t)(ratio + s) * width;
            kvst[to + c] = kvst[from + c];
            kvst[to + hd + c] = kvst[from + hd + c];
            scst[to + c] = scst[from + c];
            scst[to + hd + c] = scst[from + hd + c];
        }
    }
}

/* idxs[0, n_win): ring slots (pos - k) % win; idxs[n_win, n_win + take):
 * mode 1 every compressed row (offset + j), mode 2 the selection already
 * written there by the top-k, offset where >= 0. */
__global__ void __launch_bounds__(NR_THREADS)
k_attn_idxs(int *__restrict__ idxs, int pos, int win, int n_win, int take, int mode,
            int offset)
{
    for (int i = threadIdx.x; i < n_win + take; i += NR_THREADS) {
        if (i < n_win) {
            idxs[i] = (pos - i) % win;
        } else if (mode == 1) {
            idxs[i] = offset + (i - n_win);
        } else {
            const int v = idxs[i];
            idxs[i] = v >= 0 ? v + offset : v;
        }
    }
}

} // namespace

int dsv4_norm_rope_launch(float *dst, int dst_stride, const float *src, int src_stride,
                          const float *w, int nvec, int n, int norm, float eps, int rd,
                          const float *cs, const float *sn, int pos, int half, int inverse,
                          hipStream_t st)
{
    if (nvec <= 0 || n <= 0 || rd < 0 || rd > n || (rd & 1) || (rd && (!cs || !sn)) ||
        pos < 0 || (rd && half < rd / 2)) {
        DSV4_ERR("norm_rope: bad arguments (nvec %d n %d rd %d pos %d)", nvec, n, rd, pos);
        return -1;
    }
    hipLaunchKernelGGL(k_norm_rope, dim3(nvec), dim3(NR_THREADS), 0, st, dst, dst_stride,
                       src, src_stride, w, n, norm, eps, rd, cs, sn, pos, half, inverse);
    HIP_OK(hipGetLastError(), "norm_rope launch");
    return 0;
}

int dsv4_comp_update_launch(float *kv_row, float *score_row, const float *kv_in,
                            const float *score_in, const float *ape_row, int width,
                            hipStream_t st)
{
    if (width <= 0) return -1;
    hipLaunchKernelGGL(k_comp_update, dim3((width + NR_THREADS - 1) / NR_THREADS),
                       dim3(NR_THREADS), 0, st, kv_row, score_row, kv_in, score_in,
                       ape_row, width);
    HIP_OK(hipGetLastError(), "comp_update launch");
    return 0;
}

int dsv4_comp_pool_launch(float *out, float *kv_state, float *score_state, int ratio,
                          int hd, hipStream_t st)
{
    if (ratio <= 0 || hd <= 0) return -1;
    hipLaunchKernelGGL(k_comp_pool, dim3((hd + NR_THREADS - 1) / NR_THREADS),
                       dim3(NR_THREADS), 0, st, out, kv_state, score_state, ratio, hd,
                       ratio == 4 ? 1 : 0);
    HIP_OK(hipGetLastError(), "comp_pool launch");
    return 0;
}

int dsv4_attn_idxs_launch(int *idxs, int pos, int win, int n_win, int take, int mode,
                          int offset, hipStream_t st)
{
    if (win <= 0 || n_win < 0 || n_win > win || take < 0 || pos < 0) return -1;
    hipLaunchKernelGGL(k_attn_idxs, dim3(1), dim3(NR_THREADS), 0, st, idxs, pos, win, n_win,
                       take, mode, offset);
    HIP_OK(hipGetLastError(), "attn_idxs launch");
    return 0;
}
