/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_gpu_stub.c - the CPU-only build of include/dsv4_gpu.h.
 *
 * Replaces the reference's src/cuda/dsv4_cuda_stub.c:12-31 and, unlike it,
 * defines EVERY symbol of the header (the reference stub omits
 * dsv4_cuda_mmq_n, so a CPU-only link of dsv4_matmul.c fails). Nothing is
 * ever resident, so the dispatch's residency check sends every matrix to the
 * CPU kernels; an entry point that would need the device reports failure
 * (-1 / NULL), and the two that the reference aborts on abort.
 */
#include <stdio.h>
#include <stdlib.h>

#include "../../include/dsv4_gpu.h"

static void no_device(const char *what)
{
    fprintf(stderr, "dsv4_gpu: %s called in a build without HIP\n", what);
    abort();
}

int dsv4_gpu_available(void) { return 0; }
int dsv4_gpu_set_blocking_sync(void) { return -1; }
int dsv4_gpu_init(void) { return -1; }
size_t dsv4_gpu_free_vram(void) { return 0; }
void dsv4_gpu_shutdown(void) {}

int dsv4_gpu_upload(const DSV4QMat *m) { (void)m; return -1; }
int dsv4_gpu_upload_f32s(const DSV4QMat *m) { (void)m; return -1; }
int dsv4_gpu_has(const DSV4QMat *m) { (void)m; return 0; }
void dsv4_gpu_mmq(float *y, const float *x, const DSV4QMat *m)
{ (void)y; (void)x; (void)m; no_device("dsv4_gpu_mmq"); }
void dsv4_gpu_mmq_n(float *y, const float *x, const DSV4QMat *m, int nt)
{ (void)y; (void)x; (void)m; (void)nt; no_device("dsv4_gpu_mmq_n"); }
int dsv4_gpu_fp8_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const void *d_s, int scale_fmt, int rows, int cols,
                        void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)d_s; (void)scale_fmt; (void)rows;
  (void)cols; (void)stream; return -1; }

int dsv4_gpu_fp4_gemv_d(float *d_y, const float *d_x, const uint8_t *d_w,
                        const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c,
                        void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)d_s; (void)rows; (void)cols; (void)blk_r;
  (void)blk_c; (void)stream; return -1; }

int dsv4_gpu_bf16_gemv_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                         int cols, void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)rows; (void)cols; (void)stream; return -1; }

int dsv4_gpu_fp4_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const uint8_t *d_s, int rows, int cols, int blk_r, int blk_c, int nt,
                          void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)d_s; (void)rows; (void)cols; (void)blk_r;
  (void)blk_c; (void)nt; (void)stream; return -1; }

int dsv4_gpu_bf16_gemv_n_d(float *d_y, const float *d_x, const uint16_t *d_w, int rows,
                           int cols, int nt, void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)rows; (void)cols; (void)nt; (void)stream;
  return -1; }

int dsv4_gpu_head_argmax(const float *x, const DSV4QMat *head)
{ (void)x; (void)head; return -1; }
int dsv4_gpu_argmax_d(int *d_out, const float *d_v, int n, void *stream)
{ (void)d_out; (void)d_v; (void)n; (void)stream; return -1; }
int dsv4_gpu_embed_row_d(float *d_dst, const void *d_table, int wdt, long long row,
                         int hidden, void *stream)
{ (void)d_dst; (void)d_table; (void)wdt; (void)row; (void)hidden; (void)stream; return -1; }

dsv4_gpu_ckpt *dsv4_gpu_ckpt_open(const char *dir) { (void)dir; return NULL; }
void dsv4_gpu_ckpt_close(dsv4_gpu_ckpt *c) { (void)c; }
int dsv4_gpu_ckpt_has(const dsv4_gpu_ckpt *c, const char *name) { (void)c; (void)name; return 0; }
int dsv4_gpu_ckpt_load_qmat(dsv4_gpu_ckpt *c, const char *base, int wdt, int rows,
                            int cols, DSV4QMat *out)
{ (void)c; (void)base; (void)wdt; (void)rows; (void)cols; (void)out; return -1; }
int dsv4_gpu_ckpt_load_expert(dsv4_gpu_ckpt *c, int layer, int expert, int hidden,
                              int inter, DSV4ExpertW *out)
{ (void)c; (void)layer; (void)expert; (void)hidden; (void)inter; (void)out; return -1; }
int dsv4_gpu_ckpt_load_layer(dsv4_gpu_ckpt *c, const dsv4_gpu_ckpt_dims *d, int layer,
                             dsv4_gpu_layer_mats *out, DSV4ExpertW *experts)
{ (void)c; (void)d; (void)layer; (void)out; (void)experts; return -1; }
int dsv4_gpu_ckpt_stats_get(const dsv4_gpu_ckpt *c, dsv4_gpu_ckpt_stats *out)
{ (void)c; (void)out; return -1; }

int dsv4_gpu_dump_e4m3(float *h) { (void)h; return -1; }
int dsv4_gpu_dump_e8m0(float *h) { (void)h; return -1; }
int dsv4_gpu_dump_e2m1(float *h) { (void)h; return -1; }
int dsv4_gpu_dump_fp4_bytes(float *h) { (void)h; return -1; }
int dsv4_gpu_dump_e4m3_scaled(float *h, int e8m0) { (void)h; (void)e8m0; return -1; }

int dsv4_gpu_upload_expert(int layer, int expert, const DSV4ExpertW *e)
{ (void)layer; (void)expert; (void)e; return -1; }
int dsv4_gpu_bind_expert_d(int layer, int expert, const DSV4ExpertW *e)
{ (void)layer; (void)expert; (void)e; return -1; }
int dsv4_gpu_has_expert(int layer, int expert) { (void)layer; (void)expert; return 0; }
int dsv4_gpu_moe_fp4(float *out, const float *x, int layer, const int *idx,
                     const float *w, int topk, int hidden, int inter,
                     float swiglu_limit)
{ (void)out; (void)x; (void)layer; (void)idx; (void)w; (void)topk;
  (void)hidden; (void)inter; (void)swiglu_limit; return -1; }
int dsv4_gpu_moe_fp4_d(float *d_out, const float *d_x, int layer,
                       const int *d_idx, const float *d_w, int topk,
                       int hidden, int inter, float swiglu_limit, void *stream)
{ (void)d_out; (void)d_x; (void)layer; (void)d_idx; (void)d_w; (void)topk;
  (void)hidden; (void)inter; (void)swiglu_limit; (void)stream; return -1; }
int dsv4_gpu_moe_fp4_n(float *out, const float *x, int layer, const int *idx,
                       const float *w, int nt, int topk, int hidden, int inter,
                       float swiglu_limit)
{ (void)out; (void)x; (void)layer; (void)idx; (void)w; (void)nt; (void)topk; (void)hidden;
  (void)inter; (void)swiglu_limit; return -1; }

int dsv4_gpu_moe_fp4_n_d(float *d_out, const float *d_x, int layer, const int *d_idx,
                         const float *d_w, int nt, int topk, int hidden, int inter,
                         float swiglu_limit, void *stream)
{ (void)d_out; (void)d_x; (void)layer; (void)d_idx; (void)d_w; (void)nt; (void)topk;
  (void)hidden; (void)inter; (void)swiglu_limit; (void)stream; return -1; }

int dsv4_gpu_moe_fp4_noalloc_d(float *d_out, const float *d_x, int layer,
                               const int *d_idx, const float *d_w, int topk,
                               int hidden, int inter, float swiglu_limit, void *stream)
{ (void)d_out; (void)d_x; (void)layer; (void)d_idx; (void)d_w; (void)topk;
  (void)hidden; (void)inter; (void)swiglu_limit; (void)stream; return -1; }

dsv4_gpu_kv *dsv4_gpu_kv_create(int n_rows, int row_dim, int fmt)
{ (void)n_rows; (void)row_dim; (void)fmt; return NULL; }
int dsv4_gpu_kv_write_rows(dsv4_gpu_kv *kv, int row0, int n, const void *rows,
                           const float *row_scales)
{ (void)kv; (void)row0; (void)n; (void)rows; (void)row_scales; return -1; }
void *dsv4_gpu_kv_data(const dsv4_gpu_kv *kv) { (void)kv; return NULL; }
float *dsv4_gpu_kv_scales(const dsv4_gpu_kv *kv) { (void)kv; return NULL; }
void dsv4_gpu_kv_free(dsv4_gpu_kv *kv) { (void)kv; }

int dsv4_gpu_indexer_score(float *out, const float *q, const float *w, int H,
                           int D, const dsv4_gpu_kv *keys, int row0,
                           int key_stride, int n)
{ (void)out; (void)q; (void)w; (void)H; (void)D; (void)keys; (void)row0;
  (void)key_stride; (void)n; return -1; }
int dsv4_gpu_topk(int *idxs, const float *scores, int n, int k)
{ (void)idxs; (void)scores; (void)n; (void)k; return -1; }
int dsv4_gpu_indexer_topk(int *idxs, const float *q, const float *w, int H,
                          int D, const dsv4_gpu_kv *keys, int row0,
                          int key_stride, int n, int k)
{ (void)idxs; (void)q; (void)w; (void)H; (void)D; (void)keys; (void)row0;
  (void)key_stride; (void)n; (void)k; return -1; }
int dsv4_gpu_sparse_attn(float *o, const float *q, const dsv4_gpu_kv *kv,
                         const float *sink, const int *idxs, int h, int d_qk,
                         int d_v, int topk, float scale)
{ (void)o; (void)q; (void)kv; (void)sink; (void)idxs; (void)h; (void)d_qk;
  (void)d_v; (void)topk; (void)scale; return -1; }
int dsv4_gpu_indexer_score_d(float *d_out, const float *d_q, const float *d_w,
                             int H, int D, const void *d_keys,
                             const float *d_key_scales, int key_fmt,
                             int key_stride, int n, float scale, void *stream)
{ (void)d_out; (void)d_q; (void)d_w; (void)H; (void)D; (void)d_keys;
  (void)d_key_scales; (void)key_fmt; (void)key_stride; (void)n; (void)scale;
  (void)stream; return -1; }
int dsv4_gpu_topk_d(int *d_idxs, const float *d_scores, int n, int k,
                    void *stream)
{ (void)d_idxs; (void)d_scores; (void)n; (void)k; (void)stream; return -1; }
int dsv4_gpu_sparse_attn_d(float *d_o, const float *d_q, const void *d_kv,
                           int kv_fmt, int kv_stride, int kv_rows,
                           const float *d_sink, const int *d_idxs, int h,
                           int d_qk, int d_v, int topk, float scale,
                           void *stream)
{ (void)d_o; (void)d_q; (void)d_kv; (void)kv_fmt; (void)kv_stride;
  (void)kv_rows; (void)d_sink; (void)d_idxs; (void)h; (void)d_qk; (void)d_v;
  (void)topk; (void)scale; (void)stream; return -1; }
int dsv4_gpu_mla_decode_d(float *d_o, int *d_idxs,
                          const float *d_q_idx, const float *d_w_idx, int H,
                          int D, const void *d_keys, const float *d_key_scales,
                          int key_fmt, int key_stride, int n, int k,
                          const float *d_q, const void *d_kv, int kv_fmt,
                          int kv_stride, int kv_rows, const float *d_sink,
                          int h, int d_qk, int d_v, float attn_scale,
                          void *stream)
{ (void)d_o; (void)d_idxs; (void)d_q_idx; (void)d_w_idx; (void)H; (void)D;
  (void)d_keys; (void)d_key_scales; (void)key_fmt; (void)key_stride; (void)n;
  (void)k; (void)d_q; (void)d_kv; (void)kv_fmt; (void)kv_stride;
  (void)kv_rows; (void)d_sink; (void)h; (void)d_qk; (void)d_v;
  (void)attn_scale; (void)stream; return -1; }
int dsv4_gpu_attn_bind(int layer, const dsv4_gpu_attn_cfg *c, const dsv4_gpu_attn_w *w)
{ (void)layer; (void)c; (void)w; return -1; }
int dsv4_gpu_attn_ready(int layer) { (void)layer; return 0; }
int dsv4_gpu_attn_reset(int layer) { (void)layer; return -1; }
int dsv4_gpu_attn_step(float *out, const float *x, int layer, int pos)
{ (void)out; (void)x; (void)layer; (void)pos; return -1; }
int dsv4_gpu_attn_step_d(float *d_out, const float *d_x, int layer, int pos, void *stream)
{ (void)d_out; (void)d_x; (void)layer; (void)pos; (void)stream; return -1; }
int dsv4_gpu_fp8_gemv_n_d(float *d_y, const float *d_x, const uint8_t *d_w,
                          const void *d_s, int scale_fmt, int rows, int cols, int nt,
                          void *stream)
{ (void)d_y; (void)d_x; (void)d_w; (void)d_s; (void)scale_fmt; (void)rows; (void)cols;
  (void)nt; (void)stream; return -1; }
