/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_attnblk.hip - the small kernels of the attention block on gfx950.
 *
 * attention() (reference src/model/dsv4_layer.c:213-336) runs, for one token:
 * five to nine GEMVs (the FP8 / BF16 kernels of this library), the CSA
 * score / top-k / sparse attention (dsv4_mla.hip), and the element-wise steps
 * here:
 *   - k_block_prep: what the step needs right after the x projections, in
 *     one launch -- q's learned norm (RMSNorm, dsv4_ops.c:24-31, weighted),
 *     kv_norm + RoPE (dsv4_rope.c:105-119, interleaved pairs) into the ring
 *     slot, and
 *     the compressor's token into its slot with score + ape
 *     (dsv4_compress.c:87-98);
 *   - k_comp_close: a closing window in one launch -- the compressor's
 *     pool (dsv4_compress.c:100-137: the per-channel softmax pool over the
 *     slots; ratio 4: the previous window's first halves and the current
 *     window's second halves), the ratio-4 slide, then comp.norm and RoPE of
 *     the pooled row (dsv4_layer.c:252-255). The attention block binds
 *     compressed layers of head_dim <= 1024 only (one thread per channel).
 * The attention's row list (the window's ring slots, then the compressed
 * rows) is built inside the attention kernel (Dsv4Rows).
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

#include "dsv4_prep_rows.h"

/* The attention block's step after its x projections, in one launch:
 * workgroup j < nj runs norm job j (norm_rope_vec), the rest copy the
 * compressor's token into its slot (k_comp_update's work). The jobs touch
 * disjoint memory. */
__global__ void __launch_bounds__(NR_THREADS)
k_block_prep(Dsv4Prep a)
{
    prep_rows(a, (int)blockIdx.x);
}

/* A closing window in one launch, one workgroup, one thread per channel c
 * (blockDim >= hd): the pool of channel c over the slots (dsv4_compress.c:
 * 100-137; ratio 4 -- ov -- pools slots 0..ratio-1 from the previous
 * window's first halves, columns c, and slots ratio..2 ratio-1 from the
 * current window's second halves, columns hd + c; the slot loads of a batch
 * of 8 issued together, the arithmetic in slot order), the ratio-4 slide of
 * the current window into the previous one, then the weighted RMSNorm of the
 * pooled row and RoPE of its last rd elements at pos, written to out. */
constexpr int CC_MAX = 1024;

__global__ void __launch_bounds__(CC_MAX)
k_comp_close(float *__restrict__ out, float *__restrict__ kvst, float *__restrict__ scst,
             int ratio, int hd, int ov, const float *__restrict__ w, float eps, int rd,
             const float *__restrict__ cs, const float *__restrict__ sn, int pos, int half)
{
    __shared__ float row[CC_MAX];
    __shared__ double part[CC_MAX / 64];
    const int c = threadIdx.x;
    const bool live = c < hd;
    const int cc = live ? c : 0;
    const int width = ov ? 2 * hd : hd;
    const int slots = ov ? 2 * ratio : ratio;
    const int t0 = hd - rd;
    /* the RoPE pair's table entries and the weight, loaded with the slots */
    const int p = (c - t0) >> 1;
    const bool pr = live && c >= t0 && ((c - t0) & 1) == 0;
    float rc = 1.0f, rs = 0.0f;
    if (pr) {
        rc = cs[(size_t)pos * half + p];
        rs = sn[(size_t)pos * half + p];
    }
    const float wc = live ? w[cc] : 0.0f;
    float mx = -INFINITY;
    double den = 0.0, acc = 0.0;
    if (slots <= 8) {
        /* The window and the slide's sources in one batch of loads, all
         * issued before any store. The slide writes the arrays it reads, so
         * a load that followed one of its stores could not be moved ahead of
         * it: as a loop of copies it made one round trip per slot. ov is
         * ratio 4 (the launcher), so its 8 slots always take this path. */
        const int chi = ov ? hd + cc : cc;
        float sv[8], kv[8], ka[4], kb[4], sa[4], sb[4];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int s = min(u, slots - 1);
            const int col = (ov && s >= ratio) ? hd + cc : cc;
            sv[u] = scst[(size_t)s * width + col];
            kv[u] = kvst[(size_t)s * width + col];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t from = (size_t)min(ratio + u, slots - 1) * width;
            ka[u] = kvst[from + cc];
            kb[u] = kvst[from + chi];
            sa[u] = scst[from + cc];
            sb[u] = scst[from + chi];
        }
        for (int u = 0; u < slots; u++) if (sv[u] > mx) mx = sv[u];
        if (mx != -INFINITY)
            for (int u = 0; u < slots; u++) {
                if (sv[u] == -INFINITY) continue;
                const double e = (double)expf(sv[u] - mx);
                den += e;
                acc += e * (double)kv[u];
            }
        if (live && ov) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (u < ratio) {
                    const size_t to = (size_t)u * width;
                    kvst[to + c] = ka[u];
                    kvst[to + hd + c] = kb[u];
                    scst[to + c] = sa[u];
                    scst[to + hd + c] = sb[u];
                }
            }
        }
    } else {
        /* more slots (no slide): the max over all of them first, then the
         * weighted sum, each pass in batches of 8 loads */
        for (int s0 = 0; s0 < slots; s0 += 8) {
            float sv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int s = min(s0 + u, slots - 1);
                sv[u] = scst[(size_t)s * width + cc];
            }
            for (int u = 0; u < 8 && s0 + u < slots; u++) if (sv[u] > mx) mx = sv[u];
        }
        if (mx != -INFINITY) {
            for (int s0 = 0; s0 < slots; s0 += 8) {
                float sv[8], kv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int s = min(s0 + u, slots - 1);
                    sv[u] = scst[(size_t)s * width + cc];
                    kv[u] = kvst[(size_t)s * width + cc];
                }
                for (int u = 0; u < 8 && s0 + u < slots; u++) {
                    if (sv[u] == -INFINITY) continue;
                    const double e = (double)expf(sv[u] - mx);
                    den += e;
                    acc += e * (double)kv[u];
                }
            }
        }
    }
    const float r = (live && mx != -INFINITY) ? (float)(acc / den) : 0.0f;
    /* RMSNorm over the pooled row (sum of squares in double, a tree) */
    double sq = live ? (double)r * (double)r : 0.0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if ((c & 63) == 0) part[c >> 6] = sq;
    __syncthreads();
    double t = part[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t += part[i];
    const float inv = (float)(1.0 / sqrt(t / (double)hd + (double)eps));
    const float v = wc * (r * inv);
    row[c] = v;
    __syncthreads();
    if (!live) return;
    if (c < t0) {
        out[c] = v;
    } else if (pr) {
        const float re = v, im = row[c + 1];
        out[c] = re * rc - im * rs;
        out[c + 1] = re * rs + im * rc;
    }
}

} // namespace

int dsv4_block_prep_launch(const Dsv4Prep *a, hipStream_t st)
{
    if (a->nj < 0 || a->nj > 2 || a->width < 0 || (a->width && (!a->kvs || !a->scs))) {
        DSV4_ERR("block_prep: bad arguments (nj %d width %d)", a->nj, a->width);
        return -1;
    }
    for (int i = 0; i < a->nj; i++) {
        const Dsv4NormJob &j = a->job[i];
        if (j.n <= 0 || j.rd < 0 || j.rd > j.n || (j.rd & 1) || (j.rd && (!a->cs || !a->sn)) ||
            a->pos < 0 || (j.rd && a->half < j.rd / 2)) {
            DSV4_ERR("block_prep: bad norm job %d (n %d rd %d)", i, j.n, j.rd);
            return -1;
        }
    }
    const int nb = prep_wgs(*a);
    if (nb == 0) return 0;
    hipLaunchKernelGGL(k_block_prep, dim3(nb), dim3(NR_THREADS), 0, st, *a);
    HIP_OK(hipGetLastError(), "block_prep launch");
    return 0;
}

int dsv4_comp_close_launch(float *out, float *kv_state, float *score_state, int ratio,
                           int hd, const float *w, float eps, int rd, const float *cs,
                           const float *sn, int pos, int half, hipStream_t st)
{
    if (ratio <= 0 || hd <= 0 || hd > CC_MAX || !w || rd < 0 || rd > hd || (rd & 1) ||
        (rd && (!cs || !sn || half < rd / 2)) || pos < 0) {
        DSV4_ERR("comp_close: bad arguments (ratio %d hd %d rd %d)", ratio, hd, rd);
        return -1;
    }
    const int nt = (hd + 63) / 64 * 64;
    hipLaunchKernelGGL(k_comp_close, dim3(1), dim3(nt), 0, st, out, kv_state, score_state,
                       ratio, hd, ratio == 4 ? 1 : 0, w, eps, rd, cs, sn, pos, half);
    HIP_OK(hipGetLastError(), "comp_close launch");
    return 0;
}
