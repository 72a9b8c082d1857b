/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_oracle.c - CPU restatement of the reference decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU backend is
 * compared against. Nothing in the shipped library links it, calls it or
 * falls back to it; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.
 *
 * Every function restates one reference function from
 * ronak-create/deepseek-v4-in-c and cites the file:line it follows. The
 * arithmetic order is part of the contract (the reference is built with
 * -ffp-contract=off, and so is this file): a double fma chain, a fixed
 * 16-accumulator tree, separate multiply and add where the reference writes
 * `a += b * c`. Generalisations the hot-path configs need (fp32 block scales,
 * d_qk != d_v, an optional sink, a key stride) reduce to the reference's exact
 * loops in the special case, and the tests check that case bit for bit
 * against the compiled reference (oracle/_ref) where it is built.
 *
 * Pinning (what checks each function besides the compiled reference):
 *   decoders      closed forms over all 256/256/16 codes (test_oracle_formats)
 *   matmul fp8/4  exact-representable known answers (test_oracle_matmul)
 *   swiglu / moe  limit<=0 reduces to silu*up; k-order sum vs brute force
 *   indexer       ReLU/scale/weight/Hadamard known answers
 *   topk          ties-to-lower-index {1,2,5,3}; stable sort equivalence
 *   sparse_attn   mean, sink-halves, masks; textbook softmax when sink=-inf
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------- decoders ---
 * dsv4_quant.h:74-88 (E8M0), :101-130 (E4M3FN), :141-164 (E2M1). */
float orc_e8m0_to_f32(uint8_t b)
{
    union { uint32_t u; float f; } v;
    if (b == 0xFFu) { v.u = 0x7FC00000u; return v.f; }   /* NaN            */
    if (b == 0x00u) { v.u = 0x00400000u; return v.f; }   /* 2^-127 subnorm */
    v.u = (uint32_t)b << 23;
    return v.f;
}

float orc_e4m3_to_f32(uint8_t b)
{
    const uint32_t sign = (uint32_t)(b & 0x80u) << 24;
    const uint32_t ex = (uint32_t)(b >> 3) & 0x0Fu;
    const uint32_t mn = (uint32_t)b & 0x07u;
    union { uint32_t u; float f; } v;
    if (ex == 0) {
        if (mn == 0) { v.u = sign; return v.f; }
        /* man * 2^-9: renormalise, f32 exponent field starts at 120. */
        uint32_t m = mn, e = 120u;
        while (!(m & 0x04u)) { m <<= 1; e--; }
        v.u = sign | (e << 23) | ((m & 0x03u) << 21);
        return v.f;
    }
    if (ex == 0x0Fu && mn == 0x07u) { v.u = sign | 0x7FC00000u; return v.f; }
    v.u = sign | ((ex + 120u) << 23) | (mn << 20);
    return v.f;
}

static const float orc_e2m1_tab[16] = {
     0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f
};

float orc_e2m1_to_f32(uint8_t nib) { return orc_e2m1_tab[nib & 0x0Fu]; }

void orc_dump_e4m3(float *out256) { for (int i = 0; i < 256; i++) out256[i] = orc_e4m3_to_f32((uint8_t)i); }
void orc_dump_e8m0(float *out256) { for (int i = 0; i < 256; i++) out256[i] = orc_e8m0_to_f32((uint8_t)i); }
void orc_dump_e2m1(float *out16)  { for (int i = 0; i < 16; i++)  out16[i]  = orc_e2m1_to_f32((uint8_t)i); }

/* bf16 -> double (dsv4_matmul.c:108-112 bf16d): the 16 bits are the top half
 * of an IEEE float, widened exactly. */
static double orc_bf16_to_f64(uint16_t h)
{
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return (double)f;
}

/* One table per process; every entry is the decoder's own output. */
static float g_e4m3[256];
static int g_e4m3_ready;
static void e4m3_table(void)
{
    if (g_e4m3_ready) return;
    for (int i = 0; i < 256; i++) g_e4m3[i] = orc_e4m3_to_f32((uint8_t)i);
    g_e4m3_ready = 1;
}

/* ------------------------------------------------------- block dot tree ---
 * dsv4_matmul.c:51-64 (BLOCK_DOT_S): 16 double accumulators a[l] fed by
 * fma(w, (double)x, a[l]) in 16-wide strides, folded as
 * (a0+a4)+(a8+a12) ... then (b0+b1)+(b2+b3), then an fma tail. */
static double block_dot(const double *wv, const float *xb, int n)
{
    double a[16] = {0};
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int l = 0; l < 16; l++)
            a[l] = fma(wv[i + l], (double)xb[i + l], a[l]);
    const double b0 = (a[0] + a[4]) + (a[8] + a[12]);
    const double b1 = (a[1] + a[5]) + (a[9] + a[13]);
    const double b2 = (a[2] + a[6]) + (a[10] + a[14]);
    const double b3 = (a[3] + a[7]) + (a[11] + a[15]);
    double acc = (b0 + b1) + (b2 + b3);
    for (; i < n; i++) acc = fma(wv[i], (double)xb[i], acc);
    return acc;
}

/* The same tree over bf16 weights (widened exactly: the bf16 bits are the
 * top half of the float). */
static double bf16_dot(const uint16_t *w, const float *xb, int n)
{
    double a[16] = {0};
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int l = 0; l < 16; l++)
            a[l] = fma(orc_bf16_to_f64(w[i + l]), (double)xb[i + l], a[l]);
    const double b0 = (a[0] + a[4]) + (a[8] + a[12]);
    const double b1 = (a[1] + a[5]) + (a[9] + a[13]);
    const double b2 = (a[2] + a[6]) + (a[10] + a[14]);
    const double b3 = (a[3] + a[7]) + (a[11] + a[15]);
    double acc = (b0 + b1) + (b2 + b3);
    for (; i < n; i++) acc = fma(orc_bf16_to_f64(w[i]), (double)xb[i], acc);
    return acc;
}

/* dsv4_matmul.c:275-291 (dsv4_matmul_bf16 via GEN_MATMULS): one dot over the
 * whole row in the block-dot tree, rounded to float once. */
void orc_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out)
{
#pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++)
        y[o] = (float)bf16_dot(W + (size_t)o * in, x, in);
}

/* Scale of block (row-block rb, col-block cb): E8M0 byte (the reference's
 * format, dsv4_matmul.c:312-313) or, for the fp32-scaled configs, the float
 * itself. For a power-of-two scale the two are the same double. */
static double block_scale(const void *S, int kind, size_t at)
{
    if (kind == 0) return (double)orc_e8m0_to_f32(((const uint8_t *)S)[at]);
    return (double)((const float *)S)[at];
}

/* dsv4_matmul.c:293-318 (dsv4_matmul_fp8 via GEN_MATMULS). The scale is
 * applied once per block to the block's dot, `total += acc * s`, and the row
 * total is rounded to float once. */
void orc_matmul_fp8(float *y, const float *x, const uint8_t *W, const void *S,
                    int scale_kind, int in, int out, int blk_r, int blk_c)
{
    e4m3_table();
    const int sc = (in + blk_c - 1) / blk_c;
#pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        double wv[512];
        const uint8_t *rw = W + (size_t)o * in;
        double total = 0.0;
        for (int c0 = 0; c0 < in; c0 += blk_c) {
            const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
            double acc;
            if (n <= 512) {
                for (int i = 0; i < n; i++) wv[i] = (double)g_e4m3[rw[c0 + i]];
                acc = block_dot(wv, x + c0, n);
            } else {
                double *big = (double *)malloc((size_t)n * sizeof *big);
                for (int i = 0; i < n; i++) big[i] = (double)g_e4m3[rw[c0 + i]];
                acc = block_dot(big, x + c0, n);
                free(big);
            }
            total += acc * block_scale(S, scale_kind,
                                       (size_t)(o / blk_r) * sc + (c0 / blk_c));
        }
        y[o] = (float)total;
    }
}

/* dsv4_matmul.c:400-428: the batched form is nt independent GEMVs in the
 * same order, so it is written as exactly that. y is [nt][out]. */
void orc_matmul_fp8_n(float *y, const float *x, const uint8_t *W, const void *S,
                      int scale_kind, int in, int out, int blk_r, int blk_c,
                      int nt)
{
    for (int t = 0; t < nt; t++)
        orc_matmul_fp8(y + (size_t)t * out, x + (size_t)t * in, W, S,
                       scale_kind, in, out, blk_r, blk_c);
}

/* dsv4_matmul.c:320-345 (dsv4_matmul_fp4). Row stride in/2 bytes; element i
 * is the low nibble of byte i/2 when i is even (dsv4_quant.h:155-164). */
void orc_matmul_fp4(float *y, const float *x, const uint8_t *W,
                    const uint8_t *S, int in, int out, int blk_r, int blk_c)
{
    const int sc = (in + blk_c - 1) / blk_c;
#pragma omp parallel for schedule(static) if (out > 64)
    for (int o = 0; o < out; o++) {
        double wv[512];
        const uint8_t *row = W + (size_t)o * ((size_t)in / 2);
        double total = 0.0;
        for (int c0 = 0; c0 < in; c0 += blk_c) {
            const int n = (in - c0 < blk_c) ? (in - c0) : blk_c;
            double *buf = (n <= 512) ? wv : (double *)malloc((size_t)n * sizeof *buf);
            for (int i = 0; i < n; i++) {
                const int64_t e = (int64_t)c0 + i;
                const uint8_t byte = row[e >> 1];
                const uint8_t nib = (e & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0Fu);
                buf[i] = (double)orc_e2m1_tab[nib];
            }
            const double acc = block_dot(buf, x + c0, n);
            if (buf != wv) free(buf);
            total += acc * (double)orc_e8m0_to_f32(
                         S[(size_t)(o / blk_r) * sc + (c0 / blk_c)]);
        }
        y[o] = (float)total;
    }
}

/* dsv4_ops.c:60-78. Asymmetric clamp: up to [-L, L], gate to (-inf, L];
 * limit <= 0 disables it. silu in f32 with libm expf. */
void orc_swiglu(float *y, const float *gate, const float *up, int n, float limit)
{
    if (limit > 0.0f) {
        for (int i = 0; i < n; i++) {
            float u = up[i];
            if (u > limit) u = limit;
            if (u < -limit) u = -limit;
            float g = gate[i];
            if (g > limit) g = limit;
            const float s = g / (1.0f + expf(-g));
            y[i] = s * u;
        }
    } else {
        for (int i = 0; i < n; i++) {
            const float g = gate[i];
            y[i] = (g / (1.0f + expf(-g))) * up[i];
        }
    }
}

/* One routed expert: dsv4_layer.c:199-206 (expert_forward):
 * w2 · swiglu(w1·x, w3·x). */
void orc_expert_fp4(float *out, const float *x,
                    const uint8_t *w1, const uint8_t *s1,
                    const uint8_t *w3, const uint8_t *s3,
                    const uint8_t *w2, const uint8_t *s2,
                    int hidden, int inter, float limit)
{
    float *g = (float *)malloc((size_t)inter * sizeof *g);
    float *u = (float *)malloc((size_t)inter * sizeof *u);
    float *h = (float *)malloc((size_t)inter * sizeof *h);
    orc_matmul_fp4(g, x, w1, s1, hidden, inter, 1, 32);
    orc_matmul_fp4(u, x, w3, s3, hidden, inter, 1, 32);
    orc_swiglu(h, g, u, inter, limit);
    orc_matmul_fp4(out, h, w2, s2, inter, hidden, 1, 32);
    free(g); free(u); free(h);
}

/* The routed part of moe(): dsv4_layer.c:380 (out = 0), :466-468 (one
 * accumulator per k), :471-475 (out[i] += w_k * acc_k[i], strictly in k
 * order, multiply and add rounded separately). Expert k's tensors are
 * w1[k] ... s2[k]. acc (optional, [topk][hidden]) receives the per-k
 * expert outputs. */
void orc_moe_fp4(float *out, float *acc, const float *x,
                 const uint8_t *const *w1, const uint8_t *const *s1,
                 const uint8_t *const *w3, const uint8_t *const *s3,
                 const uint8_t *const *w2, const uint8_t *const *s2,
                 const float *wts, int topk, int hidden, int inter, float limit)
{
    float *a = acc ? acc : (float *)malloc((size_t)topk * hidden * sizeof *a);
    for (int k = 0; k < topk; k++)
        orc_expert_fp4(a + (size_t)k * hidden, x, w1[k], s1[k], w3[k], s3[k],
                       w2[k], s2[k], hidden, inter, limit);
    for (int i = 0; i < hidden; i++) out[i] = 0.0f;
    for (int k = 0; k < topk; k++) {
        const float *ak = a + (size_t)k * hidden;
        const float wk = wts[k];
        for (int i = 0; i < hidden; i++) out[i] += wk * ak[i];
    }
    if (!acc) free(a);
}

/* The routed half of moe_n (dsv4_layer.c:714-855) over nt tokens. The
 * distinct experts the batch asks for are listed in first-request order
 * (:728-739); each runs over every (token, k) routed to it (run_expert_n,
 * :681-703) into that pair's own slot of expert_acc; then each token's slots
 * are summed strictly in k order (:829-839). expert_forward_n computes each
 * pair with dsv4_mmq_n, which is bit-identical per (row, token) to dsv4_mmq
 * (dsv4_matmul.c:362-376), so a pair's slot is orc_expert_fp4 of its token.
 * Expert e's tensors are w1[e] ... s2[e]; idx and wts are [nt][topk]; x and
 * out [nt][hidden]. uniq (optional, nt * topk ints) receives the distinct
 * experts in that order; returns their count. */
int orc_moe_fp4_n(float *out, int *uniq, const float *x,
                  const uint8_t *const *w1, const uint8_t *const *s1,
                  const uint8_t *const *w3, const uint8_t *const *s3,
                  const uint8_t *const *w2, const uint8_t *const *s2,
                  const int *idx, const float *wts, int nt, int topk, int hidden,
                  int inter, float limit)
{
    const int np = nt * topk;
    int *u = (int *)malloc((size_t)np * sizeof *u);
    float *acc = (float *)malloc((size_t)np * hidden * sizeof *acc);
    int nu = 0;
    for (int p = 0; p < np; p++) {
        int seen = 0;
        for (int j = 0; j < nu; j++)
            if (u[j] == idx[p]) { seen = 1; break; }
        if (!seen) u[nu++] = idx[p];
    }
    for (int j = 0; j < nu; j++) {
        const int e = u[j];
        for (int t = 0; t < nt; t++)
            for (int k = 0; k < topk; k++)
                if (idx[(size_t)t * topk + k] == e)
                    orc_expert_fp4(acc + ((size_t)t * topk + k) * hidden,
                                   x + (size_t)t * hidden, w1[e], s1[e], w3[e], s3[e],
                                   w2[e], s2[e], hidden, inter, limit);
    }
    for (int t = 0; t < nt; t++) {
        float *o = out + (size_t)t * hidden;
        for (int i = 0; i < hidden; i++) o[i] = 0.0f;
        for (int k = 0; k < topk; k++) {
            const float *ak = acc + ((size_t)t * topk + k) * hidden;
            const float wk = wts[(size_t)t * topk + k];
            for (int i = 0; i < hidden; i++) o[i] += wk * ak[i];
        }
    }
    if (uniq) memcpy(uniq, u, (size_t)nu * sizeof *u);
    free(u);
    free(acc);
    return nu;
}

/* dsv4_indexer.c:64-85. scale = (1/sqrtf(D)) * (1/sqrtf(H)) in float; per
 * position a double total over heads of ReLU(dot) * w[h], dot an fma chain in
 * ascending c; out = (float)total * scale. Keys are rows of key_stride floats
 * (the reference passes key_stride == D). */
void orc_indexer_score(float *out, const float *q, const float *kv,
                       const float *weights, int n_heads, int head_dim,
                       int n_pos, int key_stride)
{
    const float scale = (1.0f / sqrtf((float)head_dim))
                      * (1.0f / sqrtf((float)n_heads));
#pragma omp parallel for schedule(static) if (n_pos > 1024)
    for (int t = 0; t < n_pos; t++) {
        const float *kt = kv + (size_t)t * key_stride;
        double total = 0.0;
        for (int h = 0; h < n_heads; h++) {
            const float *qh = q + (size_t)h * head_dim;
            double dot = 0.0;
            for (int c = 0; c < head_dim; c++)
                dot = fma((double)qh[c], (double)kt[c], dot);
            if (dot > 0.0) total += dot * (double)weights[h];
        }
        out[t] = (float)total * scale;
    }
}

/* dsv4_indexer.c:92-106. k passes of a running arg-max over the positions not
 * yet taken, `scores[c] > scores[best]` with best starting at the first
 * untaken c: descending, ties to the lower index, k clamped to n. The
 * reference finds "taken" by scanning the earlier picks (O(k^2 n)); a flag
 * array gives the same answer in O(k n), NaN behaviour included. */
int orc_topk(int *idxs, const float *scores, int n, int k)
{
    if (k > n) k = n;
    if (k <= 0) return k;
    unsigned char *taken = (unsigned char *)calloc((size_t)n, 1);
    for (int i = 0; i < k; i++) {
        int best = -1;
        for (int c = 0; c < n; c++) {
            if (taken[c]) continue;
            if (best < 0 || scores[c] > scores[best]) best = c;
        }
        idxs[i] = best;
        taken[best] = 1;
    }
    free(taken);
    return k;
}

/* dsv4_indexer.c:113-117 and :123, dsv4_attn.c:118-128: index plumbing. */
void orc_indexer_offset(int *idxs, int n, int offset)
{
    for (int i = 0; i < n; i++) if (idxs[i] >= 0) idxs[i] += offset;
}
int orc_indexer_navail(int pos, int ratio) { return (pos + 1) / ratio; }
int orc_window_idxs(int *idxs, int pos, int win)
{
    int n = pos + 1;
    if (n > win) n = win;
    for (int k = 0; k < win; k++) idxs[k] = -1;
    for (int k = 0; k < n; k++) idxs[k] = (pos - k) % win;
    return n;
}

/* dsv4_attn.c:60-108. Per head: s_j = (float)(fma chain of q.kv) * scale, or
 * -inf for a masked (-1) slot; mx over valid s_j; e_j = expf(s_j - mx);
 * denom = sum_j (double)e_j + (double)expf(sink - mx) (the sink enters the
 * denominator only and takes no part in the max); o = sum_j e_j * kv_j in
 * f32, in j order, skipping e_j == 0; o *= (float)(1/denom).
 * Generalised: q rows are d_qk wide, kv rows kv_stride wide, the score uses
 * the first d_qk columns and the value the first d_v; sink may be NULL (no
 * sink term). d_qk == d_v == kv_stride with a sink is the reference call. */
void orc_sparse_attn(float *o, const float *q, const float *kv, int kv_stride,
                     const float *sink, const int *idxs, int h, int d_qk,
                     int d_v, int topk, float scale)
{
#pragma omp parallel for schedule(static) if (h > 4)
    for (int i = 0; i < h; i++) {
        float *s = (float *)malloc((size_t)(topk > 0 ? topk : 1) * sizeof *s);
        const float *qi = q + (size_t)i * d_qk;
        float mx = -INFINITY;
        for (int j = 0; j < topk; j++) {
            const int idx = idxs[j];
            if (idx < 0) { s[j] = -INFINITY; continue; }
            const float *kvj = kv + (size_t)idx * kv_stride;
            double acc = 0.0;
            for (int c = 0; c < d_qk; c++)
                acc = fma((double)qi[c], (double)kvj[c], acc);
            s[j] = (float)acc * scale;
            if (s[j] > mx) mx = s[j];
        }
        double denom = 0.0;
        for (int j = 0; j < topk; j++) {
            if (idxs[j] < 0) { s[j] = 0.0f; continue; }
            s[j] = expf(s[j] - mx);
            denom += (double)s[j];
        }
        if (sink) denom += (double)expf(sink[i] - mx);
        float *oi = o + (size_t)i * d_v;
        for (int c = 0; c < d_v; c++) oi[c] = 0.0f;
        for (int j = 0; j < topk; j++) {
            const int idx = idxs[j];
            if (idx < 0) continue;
            const float w = s[j];
            if (w == 0.0f) continue;
            const float *kvj = kv + (size_t)idx * kv_stride;
            for (int c = 0; c < d_v; c++) oi[c] += w * kvj[c];
        }
        const float inv = (float)(1.0 / denom);
        for (int c = 0; c < d_v; c++) oi[c] *= inv;
        free(s);
    }
}

/* ------------------------------------------------------------------ head --- */
/* The greedy pick of the decode loop (dsv4_run.c:471-472): the first index
 * of the maximum under `>`; a NaN is never chosen unless it is at index 0. */
int orc_argmax(const float *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* dsv4_embed_row (include/dsv4/dsv4.h:300-314): a BF16 row widened (the 16
 * bits become the top half of the float), or an f32 row copied. wdt 1 =
 * BF16, otherwise f32. */
void orc_embed_row(float *dst, const void *table, int wdt, long long row, int hidden)
{
    if (wdt == 1) {
        const uint16_t *p = (const uint16_t *)table + row * hidden;
        for (int i = 0; i < hidden; i++) {
            const uint32_t u = (uint32_t)p[i] << 16;
            memcpy(&dst[i], &u, sizeof u);
        }
    } else {
        const float *p = (const float *)table + row * hidden;
        for (int i = 0; i < hidden; i++) dst[i] = p[i];
    }
}

/* ------------------------------------------------------ attention block ---
 * The pieces of attention() (dsv4_layer.c:213-336) around the CSA calls:
 * RMSNorm, the per-head norm of q, RoPE and the KV compressor. */

/* dsv4_rmsnorm, dsv4_ops.c:24-31: the sum of squares in double, eps added to
 * the MEAN, y = w * (x * inv) with inv rounded to float. y may alias x. */
void orc_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    double sq = 0.0;
    for (int i = 0; i < n; i++) sq += (double)x[i] * (double)x[i];
    const float inv = (float)(1.0 / sqrt(sq / (double)n + (double)eps));
    for (int i = 0; i < n; i++) y[i] = w[i] * (x[i] * inv);
}

/* dsv4_rope_apply, dsv4_rope.c:105-119: the last rd elements of v rotated as
 * interleaved pairs (v[2i], v[2i+1]) by the table row at pos; inverse
 * negates the sine (the output de-rotation). */
void orc_rope_apply(float *v, int head_dim, int rd, const float *cs, const float *sn,
                    int pos, int table_half, int inverse)
{
    float *t = v + (head_dim - rd);
    for (int i = 0; i < rd / 2; i++) {
        const float c = cs[(size_t)pos * table_half + i];
        const float s0 = sn[(size_t)pos * table_half + i];
        const float s = inverse ? -s0 : s0;
        const float re = t[2 * i], im = t[2 * i + 1];
        t[2 * i] = re * c - im * s;
        t[2 * i + 1] = re * s + im * c;
    }
}

/* The per-head step of attention() on q (dsv4_layer.c:223-231): each head
 * scaled by 1/sqrt(mean square + eps) with no weight, then RoPE at pos. */
void orc_head_norm_rope(float *q, int H, int hd, int rd, float eps, const float *cs,
                        const float *sn, int pos)
{
    for (int h = 0; h < H; h++) {
        float *qh = q + (size_t)h * hd;
        double sq = 0.0;
        for (int i = 0; i < hd; i++) sq += (double)qh[i] * qh[i];
        const float inv = (float)(1.0 / sqrt(sq / (double)hd + (double)eps));
        for (int i = 0; i < hd; i++) qh[i] *= inv;
        orc_rope_apply(qh, hd, rd, cs, sn, pos, rd / 2, 0);
    }
}

/* One channel of the compressor's pool (dsv4_compress.c:45-63): a softmax
 * over the slots (max in float, -inf slots skipped), sums in double. */
static float pool_one(const float *kv, const float *sc, int slots, int kv_stride,
                      int sc_stride, int c)
{
    float mx = -INFINITY;
    for (int s = 0; s < slots; s++) {
        const float v = sc[(size_t)s * sc_stride + c];
        if (v > mx) mx = v;
    }
    if (mx == -INFINITY) return 0.0f;
    double den = 0.0, acc = 0.0;
    for (int s = 0; s < slots; s++) {
        const float v = sc[(size_t)s * sc_stride + c];
        if (v == -INFINITY) continue;
        const double e = (double)expf(v - mx);
        den += e;
        acc += e * (double)kv[(size_t)s * kv_stride + c];
    }
    return (float)(acc / den);
}

/* dsv4_compress_step, dsv4_compress.c:77-137 (the decode path). The token
 * goes into slot pos % ratio (ratio + pos % ratio when ratio == 4, whose
 * first `ratio` slots hold the previous window) with score + ape[pos %
 * ratio]; when the window closes, out[hd] is the per-channel pool -- over
 * `ratio` slots of width hd, or for ratio 4 over the previous window's first
 * halves then the current window's second halves -- and the ratio-4 state
 * slides down by one window. Returns 1 when out was written. score_state
 * starts at -inf. */
int orc_compress_step(float *out, const float *kv_in, const float *score_in,
                      const float *ape, float *kv_state, float *score_state, int pos,
                      int ratio, int hd)
{
    const int ov = ratio == 4, width = (1 + ov) * hd, ph = pos % ratio;
    const int slot = ov ? ratio + ph : ph;
    for (int c = 0; c < width; c++) {
        kv_state[(size_t)slot * width + c] = kv_in[c];
        score_state[(size_t)slot * width + c] = score_in[c] + ape[(size_t)ph * width + c];
    }
    if ((pos + 1) % ratio != 0) return 0;
    if (!ov) {
        for (int c = 0; c < hd; c++)
            out[c] = pool_one(kv_state, score_state, ratio, width, width, c);
        return 1;
    }
    float *gk = malloc(sizeof(float) * 2 * ratio * hd);
    float *gs = malloc(sizeof(float) * 2 * ratio * hd);
    if (!gk || !gs) { free(gk); free(gs); return -1; }
    for (int s = 0; s < 2 * ratio; s++) {
        const size_t src = (size_t)s * width + (s < ratio ? 0 : hd);
        memcpy(gk + (size_t)s * hd, kv_state + src, sizeof(float) * hd);
        memcpy(gs + (size_t)s * hd, score_state + src, sizeof(float) * hd);
    }
    for (int c = 0; c < hd; c++) out[c] = pool_one(gk, gs, 2 * ratio, hd, hd, c);
    free(gk);
    free(gs);
    memmove(kv_state, kv_state + (size_t)ratio * width, sizeof(float) * ratio * width);
    memmove(score_state, score_state + (size_t)ratio * width, sizeof(float) * ratio * width);
    return 1;
}

/* dsv4_compress_rope_pos, dsv4_compress.c:141: a compressed row is stamped
 * with the first position of the window it summarises. */
int orc_compress_rope_pos(int pos, int ratio) { return pos + 1 - ratio; }
