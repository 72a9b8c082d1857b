/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_internal.h - host-side launchers shared between the kernel files and
 * the C-ABI layer. Not installed; the public surface is include/dsv4_gpu.h. */
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/dsv4_gpu.h"

#define DSV4_ERR(...) do { fprintf(stderr, "dsv4_gpu: " __VA_ARGS__); \
                           fputc('\n', stderr); } while (0)

#define HIP_OK(call, what)                                                   \
    do {                                                                     \
        const hipError_t e_ = (call);                                        \
        if (e_ != hipSuccess) {                                              \
            DSV4_ERR("%s: %s", (what), hipGetErrorString(e_));               \
            return -1;                                                       \
        }                                                                    \
    } while (0)

/* Bytes of LDS one workgroup may use on the current device (the gfx950
 * reports 160 KiB; 64 KiB if the query fails). */
size_t dsv4_lds_limit(void);

/* Opt a kernel in to `bytes` of dynamic LDS per workgroup, at most what its
 * static LDS leaves of the device's limit. true, or false with a message
 * naming `what` when the runtime refuses; the error is cleared, and a launch
 * that needed the opt-in then fails on its own check. Callers make the
 * attempt once (a once-flag set after it, whatever the result), so a refusal
 * is reported once. */
bool dsv4_lds_optin(const void *kernel, size_t bytes, const char *what);

/* Block-scaled FP8 GEMV. sfmt 0 = E8M0 bytes, 1 = fp32. S is the scale grid
 * ceil(rows/blk_r) x sc with sc = ceil(cols/blk_c). Returns 0 / -1. valu:
 * the VALU form even for E8M0 scales, for a caller whose results need not
 * share the bits of the batched form (the attention block's projections);
 * at batch 1 it is the faster form at every E8M0 shape measured. */
int dsv4_fp8_gemv_launch(float *y, const float *x, const uint8_t *W,
                         const void *S, int sfmt, int rows, int cols,
                         int blk_r, int blk_c, hipStream_t st, bool valu = false);

/* The matrix-core form of the FP8 GEMV for E8M0-scaled matrices
 * (dsv4_fp8_mx.hip): one launch of n GEMVs that read x + i * x_stride (or,
 * listed, n matrices reading the same x), each row's bits those of the
 * batched form below for the same token. */
struct Dsv4Fp8Mx {
    float *y = nullptr;
    const float *x = nullptr;
    const uint8_t *w = nullptr, *s = nullptr;
    int rows = 0, cols = 0, sc = 0, blk_r = 128, blk_c = 128;
    /* set by dsv4_fp8_mx_launch: ceil(2^32 / blk_c), the launch shape */
    uint32_t bc_m = 0;
    int wpt = 1, spw = 1, tpw = 1, xp = 0, gx = 1, npb = 1;
    size_t lds = 0;
    int n = 1;
    long long x_stride = 0, y_stride = 0, w_stride = 0, s_stride = 0;
    int list = 0;
    const uint8_t *wl[4] = {}, *sl[4] = {};
    float *yl[4] = {};
    int rl[4] = {};
};
/* The shapes the matrix-core form takes: E8M0 scales (sfmt 0), cols a
 * multiple of 16 up to 16384, blk_c a multiple of 16. */
bool dsv4_fp8_mx_ok(int sfmt, int cols, int blk_r, int blk_c);
int dsv4_fp8_mx_launch(const Dsv4Fp8Mx &a, hipStream_t st);
/* The batched matrix-core form: y[nt][rows], x[nt][cols]; every (row,
 * token) has the bits of dsv4_fp8_mx_launch on that token. xscratch
 * (optional, dsv4_fp8_mxn_scratch_bytes of device memory): x is split into
 * its bf16 terms there once, instead of in every workgroup. */
size_t dsv4_fp8_mxn_scratch_bytes(int cols, int nt);
int dsv4_fp8_mxn_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S, int rows,
                        int cols, int blk_r, int blk_c, int nt, hipStream_t st,
                        void *xscratch = nullptr);

/* MXFP4 GEMV (dsv4_matmul_fp4): W e2m1 nibbles [rows][cols/2], S E8M0 bytes
 * [ceil(rows/blk_r)][ceil(cols/blk_c)]. _ok: the shapes it takes (cols a
 * multiple of 32 up to 16384, blk_c a multiple of 32). Returns 0 / -1. */
/* `groups` GEMVs of one shape in one launch: group i reads x + i*x_stride
 * floats, W + i*w_stride bytes and its scales at S + i*s_stride bytes, and
 * writes y + i*y_stride floats; each group's rows get the bits of a plain
 * launch on those pointers. */
int dsv4_fp8_gemv_groups_launch(float *y, const float *x, const uint8_t *W,
                                const void *S, int sfmt, int rows, int cols, int blk_r,
                                int blk_c, int groups, long long y_stride,
                                long long x_stride, long long w_stride,
                                long long s_stride, hipStream_t st, bool valu = false);

/* Up to four FP8 matrices of one width, scale format and blocking that read
 * the same x, in one launch: y[i] = W[i] x over rows[i] rows, each with the
 * bits of its own plain launch. */
int dsv4_fp8_gemv_list_launch(const float *x, int cols, int sfmt, int blk_r, int blk_c,
                              int n, const uint8_t *const *W, const void *const *S,
                              float *const *y, const int *rows, hipStream_t st,
                              bool valu = false);

/* Up to four FP8 matrices (one scale format and blocking, the VALU form)
 * and up to four BF16 matrices, all of width cols and reading the same x,
 * in one launch where the shapes take it (else a listed launch of each);
 * every row has the bits of its own GEMV. */
int dsv4_xproj_launch(const float *x, int cols, int sfmt, int blk_r, int blk_c, int nf,
                      const uint8_t *const *Wf, const void *const *Sf, float *const *yf,
                      const int *rf, int nb, const uint16_t *const *Wb, float *const *yb,
                      const int *rb, hipStream_t st);

/* The same for up to four BF16 matrices of one width. */
int dsv4_bf16_gemv_list_launch(const float *x, int cols, int n, const uint16_t *const *W,
                               float *const *y, const int *rows, hipStream_t st);

bool dsv4_fp4_gemv_ok(int rows, int cols, int blk_r, int blk_c);
int dsv4_fp4_gemv_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S,
                         int rows, int cols, int blk_r, int blk_c, hipStream_t st);
/* Batched: y[nt][rows] for x[nt][cols], every (row, token) bit-identical to
 * dsv4_fp4_gemv_launch on that token; the weights are read once. */
int dsv4_fp4_gemv_n_launch(float *y, const float *x, const uint8_t *W, const uint8_t *S,
                           int rows, int cols, int blk_r, int blk_c, int nt, hipStream_t st);

/* BF16 GEMV (dsv4_matmul_bf16): W bf16 [rows][cols]. _ok: the shapes it
 * takes (cols a multiple of 8 up to 16384). Returns 0 / -1. */
bool dsv4_bf16_gemv_ok(int rows, int cols);
int dsv4_bf16_gemv_launch(float *y, const float *x, const uint16_t *W, int rows, int cols,
                          hipStream_t st);
/* Batched: y[nt][rows] for x[nt][cols], every (row, token) bit-identical to
 * dsv4_bf16_gemv_launch on that token; the weights are read once. */
int dsv4_bf16_gemv_n_launch(float *y, const float *x, const uint16_t *W, int rows, int cols,
                            int nt, hipStream_t st);

/* Greedy argmax (the first index of the maximum, dsv4_run.c:471-472) over
 * d_v[n] into d_out[0]; scratch of dsv4_argmax_scratch_bytes. 0 / -1. */
size_t dsv4_argmax_scratch_bytes(void);
int dsv4_argmax_launch(int *d_out, const float *d_v, int n, void *scratch, hipStream_t st);

/* dsv4_embed_row (dsv4.h:300-314) on device buffers. 0 / -1. */
int dsv4_embed_row_launch(float *d_dst, const void *d_table, int wdt, long long row,
                          int hidden, hipStream_t st);

/* Batched: y[nt][rows], x[nt][cols]; per (row, token) bit-identical to the
 * GEMV above. xscratch: device memory of dsv4_fp8_n_scratch_bytes(rows, cols,
 * nt) bytes, for the E8M0 matrix-core form's split of x or the f32
 * matrix-core form's part sums (without it those forms fall back to kernels
 * that need none, with the same bits). */
size_t dsv4_fp8_n_scratch_bytes(int rows, int cols, int nt);
int dsv4_fp8_gemv_n_launch(float *y, const float *x, const uint8_t *W,
                           const void *S, int sfmt, int rows, int cols,
                           int blk_r, int blk_c, int nt, hipStream_t st,
                           void *xscratch = nullptr);

/* A matrix whose bytes are in HBM already (m->w / m->s device addresses,
 * e.g. read there from a checkpoint) made resident under those addresses;
 * `owned` (may be nullptr) is freed at shutdown. 0 / -1. */
int dsv4_res_adopt(const DSV4QMat *m, void *owned);

/* The same for a routed expert (FP4, 1x32 blocks): registered for the fused
 * MoE by (layer, expert) and its three matrices made resident. 0 / -1. */
int dsv4_expert_adopt(int layer, int expert, const DSV4ExpertW *e, void *owned);
/* The routed-expert pass's arrival counters on the current device
 * (DSV4_MOE_SYNC_WORDS words, zero between calls; nullptr before
 * dsv4_gpu_init). Calls of the pass that overlap on one device race. */
#define DSV4_MOE_SYNC_WORDS 66
uint32_t *dsv4_moe_sync(void);
/* Their undo, for a load that fails partway: the matrix keyed at `key` (or
 * the expert) leaves the tables and what it owned is freed. 0 / -1. */
int dsv4_res_release(const void *key);
int dsv4_expert_release(int layer, int expert);

/* One routed expert's device tensors (FP4 nibbles + E8M0 per 1x32). */
struct Dsv4ExpertDev {
    const uint8_t *w1, *s1, *w3, *s3, *w2, *s2;
};

/* Device scratch dsv4_moe_fp4_launch needs, in bytes (0: shape not
 * supported). */
size_t dsv4_moe_scratch_bytes(int topk, int hidden, int inter);

/* Routed MoE on the device. d_table: device array [n_table] of expert
 * tensors for this layer; d_idx/d_w device [topk]; scratch of
 * dsv4_moe_scratch_bytes. Picks the matrix-core form (dsv4_moe_mx.hip) when
 * hidden and inter are multiples of 128, else the VALU form (dsv4_moe.hip).
 * Calls that overlap on one scratch buffer race. */
int dsv4_moe_fp4_launch(float *d_out, const float *d_x,
                        const Dsv4ExpertDev *d_table, int n_table,
                        const int *d_idx, const float *d_w, int topk,
                        int hidden, int inter, float limit, void *scratch,
                        hipStream_t st);

/* Batched routed MoE (prefill, the routed half of moe_n): d_out[nt][hidden]
 * for d_x[nt][hidden], routing d_idx/d_w [nt][topk]; each distinct expert's
 * weights stream once for the batch and every token's row is bit-identical
 * to dsv4_moe_fp4_launch on that token. Scratch of dsv4_moe_n_scratch_bytes
 * (at least dsv4_moe_scratch_bytes). */
size_t dsv4_moe_n_scratch_bytes(int nt, int topk, int hidden, int inter);
int dsv4_moe_fp4_n_launch(float *d_out, const float *d_x, const Dsv4ExpertDev *d_table,
                          int n_table, const int *d_idx, const float *d_w, int nt, int topk,
                          int hidden, int inter, float limit, void *scratch, hipStream_t st);

/* The VALU form; hbuf is device scratch [topk][inter] f32. */
int dsv4_moe_fp4_valu_launch(float *d_out, const float *d_x,
                             const Dsv4ExpertDev *d_table, int n_table,
                             const int *d_idx, const float *d_w, int topk,
                             int hidden, int inter, float limit, float *hbuf,
                             hipStream_t st);

/* Index scratch (the top-k's histogram, candidates and lists) for a top-k
 * over n scores, in bytes. The standalone score needs none. */
size_t dsv4_index_scratch_bytes(int n);

/* The largest k a device top-k takes (dsv4_topk_launch refuses more). */
int dsv4_topk_kmax(void);

/* The most selected rows dsv4_attn_block_launch takes at this KV format and
 * width (0: the width is not supported). */
int dsv4_attn_max_rows(int kv_fmt, int d_qk, int d_v);

/* Whether a top-k of k over n scores starts from the level-1 histogram that
 * dsv4_indexer_score_launch builds with with_hist set. */
int dsv4_topk_takes_hist(int n, int k);

int dsv4_indexer_score_launch(float *d_out, const float *d_q, const float *d_w,
                              int H, int D, const void *d_keys,
                              const float *d_key_scales, int key_fmt,
                              int key_stride, int n, float scale, void *scratch,
                              int with_hist, hipStream_t st);

/* hist_ready: the score kernel left the level-1 histogram for these scores in
 * the scratch (only when dsv4_topk_takes_hist(n, k)). */
int dsv4_topk_launch(int *d_idxs, const float *d_scores, int n, int k,
                     void *scratch, int hist_ready, hipStream_t st);

/* Scratch needed by dsv4_attn_launch, in bytes (0: shape not supported). */
size_t dsv4_attn_scratch_bytes(int h, int d_qk, int d_v, int topk, int kv_fmt);

/* The attention block's row list, built inside the attention kernel
 * instead of in memory: rows j < n_win are the ring slots (pos - j) % win,
 * then mode 1 takes offset + (j - n_win) (every compressed row) and mode 2
 * takes d_idxs[j - n_win] + offset (the top-k's selection; negative entries
 * stay negative and are skipped). on == 0: d_idxs[j] as given. */
struct Dsv4Rows {
    int on = 0;
    int win = 0, n_win = 0, pos = 0, mode = 0, offset = 0;
};

/* The attention block's form: q_norm scales each head of q by 1/sqrt(mean
 * square + q_eps) and rope_dim > 0 RoPEs its last rope_dim elements at
 * rope_pos before the scores (dsv4_layer.c:223-231), and de-rotates the
 * output's last rope_dim elements after them (:304-305) -- on the kernels'
 * own copies; d_q is not written. rows: the row list as above (nullptr:
 * d_idxs as given). */
int dsv4_attn_block_launch(float *d_o, const float *d_q, const void *d_kv,
                           int kv_fmt, int kv_stride, int kv_rows,
                           const float *d_sink, const int *d_idxs, int h, int d_qk,
                           int d_v, int topk, float scale, void *scratch, int q_norm,
                           float q_eps, const float *rope_cs, const float *rope_sn,
                           int rope_pos, int rope_half, int rope_dim, hipStream_t st,
                           const Dsv4Rows *rows = nullptr);

/* The indexer score with its q RoPE'd at rope_pos first (rope_dim 0: as
 * given), on the kernel's own copy. */
int dsv4_indexer_score_rope_launch(float *d_out, const float *d_q, const float *d_w,
                                   int H, int D, const void *d_keys,
                                   const float *d_key_scales, int key_fmt,
                                   int key_stride, int n, float scale, void *scratch,
                                   int with_hist, const float *rope_cs,
                                   const float *rope_sn, int rope_pos, int rope_half,
                                   int rope_dim, hipStream_t st);

/* Rows outside [0, kv_rows) are treated as masked (never read). */
int dsv4_attn_launch(float *d_o, const float *d_q, const void *d_kv,
                     int kv_fmt, int kv_stride, int kv_rows,
                     const float *d_sink, const int *d_idxs, int h, int d_qk,
                     int d_v, int topk, float scale, void *scratch,
                     hipStream_t st);

/* ---- the attention block's element-wise steps (dsv4_attnblk.hip) ------ */

/* One RMSNorm (+ RoPE of the last rd elements at pos) of the block prep. */
struct Dsv4NormJob {
    float *dst;
    const float *src;
    const float *w;
    int n, rd;
};
/* The attention block's prep launch: up to two norm jobs (weighted RMSNorm,
 * optional RoPE, eps and the RoPE table shared) and the compressor's slot
 * update (kvs = kv_in, scs = sc_in + apr over width; width 0 for none). */
struct Dsv4Prep {
    Dsv4NormJob job[2];
    int nj;
    float eps;
    const float *cs, *sn;
    int pos, half;
    float *kvs, *scs;
    const float *kv_in, *sc_in, *apr;
    int width;
};
int dsv4_block_prep_launch(const Dsv4Prep *a, hipStream_t st);

/* The block's q GEMVs (up to four FP8 matrices of width cols reading qr,
 * the VALU form) and its prep step in one launch where the shapes take it:
 * each GEMV workgroup applies the q job -- qr's weighted RMSNorm (nw, eps),
 * norm_rope_vec's arithmetic -- to its own copy of qr (qr is not written),
 * and prep's at most one norm job and compressor slot run beside them.
 * Otherwise the prep launch with the q job first, then the listed GEMV;
 * the same bits either way. */
int dsv4_qproj_launch(const float *qr, int cols, const float *nw, float eps, int sfmt,
                      int blk_r, int blk_c, int nf, const uint8_t *const *Wf,
                      const void *const *Sf, float *const *yf, const int *rf,
                      const Dsv4Prep *prep, hipStream_t st);

/* A closing window in one launch (hd <= 1024): the pool (with the ratio-4
 * slide), then the weighted RMSNorm of the pooled row and RoPE of its last rd
 * elements at table row pos, into out[hd]. */
int dsv4_comp_close_launch(float *out, float *kv_state, float *score_state, int ratio,
                           int hd, const float *w, float eps, int rd, const float *cs,
                           const float *sn, int pos, int half, hipStream_t st);
