/* SPDX-License-Identifier: Apache-2.0 */
/* attn_block.c - the device attention block against the reference's own
 * attention(), layer by layer, on the tiny checkpoint.
 *
 * TEST INFRASTRUCTURE ONLY. attention() is static in the reference
 * (src/model/dsv4_layer.c:213-336), so this driver #includes that file as it
 * lies under /root/reference and calls it directly; oracle/Makefile compiles
 * it with the reference's other model sources into oracle/_ref/dsv4_attn.
 * Nothing of the reference is copied.
 *
 * For every layer of the checkpoint (compress ratios 0, 4 with the indexer,
 * and 8), fresh layer state, positions 0 .. n-1, one seeded N(0,1) input per
 * position:
 *   pass 1: the reference's attention() with every matmul on its CPU path
 *           (nothing resident yet);
 *   pass 2: the layer's matrices made resident, dsv4_gpu_attn_bind, then
 *           dsv4_gpu_attn_step per position -- the whole block on the device.
 * Prints the vector-scaled relative error per layer and position and a
 * summary; exit 0 when every step is within --tol (default 1e-4), 1
 * otherwise, 2 when no GPU is available.
 *
 * usage: dsv4_attn CKPT_DIR [N_POSITIONS] [--tol T]
 */
#include "dsv4_layer.c"

#include "dsv4_cfg.h"
#include "dsv4_gpu.h"
#include "dsv4_st.h"

void dsv4_rope_table(float *cs, float *sn, int rd, int maxpos, int orig_ctx, double theta,
                     double factor, double beta_fast, double beta_slow);

/* splitmix64 -> Box-Muller: the inputs, reproducible per (layer, pos). */
static uint64_t sm64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void normal_vec(float *v, int n, uint64_t seed)
{
    uint64_t s = seed;
    for (int i = 0; i < n; i += 2) {
        const double u1 = ((sm64(&s) >> 11) + 1.0) / 9007199254740993.0;
        const double u2 = (sm64(&s) >> 11) / 9007199254740992.0;
        const double r = sqrt(-2.0 * log(u1));
        v[i] = (float)(r * cos(2.0 * M_PI * u2));
        if (i + 1 < n) v[i + 1] = (float)(r * sin(2.0 * M_PI * u2));
    }
}

/* Vector-scaled relative error (tests/unit/test_cuda.c:160-167). */
static double vec_rel(const float *got, const float *ref, int n)
{
    double sq = 0.0;
    for (int i = 0; i < n; i++) sq += (double)ref[i] * ref[i];
    const double rms = sqrt(sq / n);
    double worst = 0.0;
    for (int i = 0; i < n; i++) {
        double s = fabs((double)ref[i]);
        if (fabs((double)got[i]) > s) s = fabs((double)got[i]);
        if (rms > s) s = rms;
        const double r = s > 0 ? fabs((double)got[i] - ref[i]) / s : 0.0;
        if (r > worst) worst = r;
    }
    return worst;
}

static int upload(const DSV4QMat *m)
{
    if (!m || !m->w) return 0;
    return dsv4_gpu_upload(m) == 0 ? 1 : -1;
}

int main(int argc, char **argv)
{
    if (argc < 2) {
        fprintf(stderr, "usage: %s CKPT_DIR [N_POSITIONS] [--tol T]\n", argv[0]);
        return 1;
    }
    int n = 40;
    double tol = 1e-4;
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--tol") && i + 1 < argc) tol = atof(argv[++i]);
        else n = atoi(argv[i]);
    }
    char path[1024];
    DSV4Cfg c;
    int cr[DSV4_MAX_LAYERS];
    snprintf(path, sizeof path, "%s/config.json", argv[1]);
    if (!dsv4_cfg_load_file(&c, cr, DSV4_MAX_LAYERS, path)) return 1;
    DSV4St st;
    if (dsv4_st_open(&st, argv[1]) != 0) return 1;
    DSV4LayerBind *lb = calloc((size_t)c.n_layers, sizeof *lb);
    for (int L = 0; L < c.n_layers; L++)
        if (dsv4_bind_layer(&st, &c, L, &lb[L]) != 0) return 1;

    const int maxpos = n + 16, half = c.qk_rope / 2, hd = c.head_dim;
    float *cs_d = malloc((size_t)maxpos * half * 4), *sn_d = malloc((size_t)maxpos * half * 4);
    float *cs_c = malloc((size_t)maxpos * half * 4), *sn_c = malloc((size_t)maxpos * half * 4);
    dsv4_rope_table(cs_d, sn_d, c.qk_rope, maxpos, 0, c.rope_theta, c.yarn_factor,
                    c.yarn_beta_fast, c.yarn_beta_slow);
    dsv4_rope_table(cs_c, sn_c, c.qk_rope, maxpos, c.yarn_orig_ctx, c.compress_rope_theta,
                    c.yarn_factor, c.yarn_beta_fast, c.yarn_beta_slow);
    DSV4Scratch s;
    if (dsv4_scratch_init(&s, &c, maxpos) != 0) return 1;

    const size_t per = (size_t)n * c.hidden;
    float *x = malloc(per * c.n_layers * sizeof(float));
    float *ref = malloc(per * c.n_layers * sizeof(float));
    float *got = malloc(per * sizeof(float));
    if (!x || !ref || !got) return 1;
    for (int L = 0; L < c.n_layers; L++)
        for (int p = 0; p < n; p++)
            normal_vec(x + (size_t)L * per + (size_t)p * c.hidden, c.hidden,
                       0x5EEDull * 1000003ull + (uint64_t)L * 4096 + (uint64_t)p);

    /* pass 1: the reference, every matmul on the CPU */
    for (int L = 0; L < c.n_layers; L++) {
        const int comp = dsv4_compress_ratio(&c, L) != 0;
        DSV4LayerState ls;
        if (dsv4_state_init(&ls, &c, L, maxpos) != 0) return 1;
        for (int p = 0; p < n; p++) {
            const int n_idx = dsv4_window_idxs(s.idxs, p, c.sliding_window);
            attention(ref + (size_t)L * per + (size_t)p * c.hidden,
                      x + (size_t)L * per + (size_t)p * c.hidden, &lb[L].w, &c, &s, &ls,
                      comp ? cs_c : cs_d, comp ? sn_c : sn_d, p, n_idx);
        }
        dsv4_state_free(&ls);
    }

    /* pass 2: the block on the device */
    if (!dsv4_gpu_available() || dsv4_gpu_init() != 0) {
        fprintf(stderr, "attn: no GPU\n");
        return 2;
    }
    double worst_all = 0.0;
    int bad = 0, steps = 0;
    for (int L = 0; L < c.n_layers; L++) {
        const DSV4AttnW *a = &lb[L].w.attn;
        const int ratio = dsv4_compress_ratio(&c, L), comp = ratio != 0;
        const DSV4QMat *m[9] = {&a->wq_a, &a->wq_b, &a->wkv, &a->wo_a, &a->wo_b,
                                a->has_comp ? &a->comp.wkv : NULL,
                                a->has_comp ? &a->comp.wgate : NULL,
                                a->has_idx ? &a->idx.wq_b : NULL,
                                a->has_idx ? &a->idx.weights_proj : NULL};
        for (int k = 0; k < 9; k++)
            if (upload(m[k]) < 0) { fprintf(stderr, "attn: upload %d of layer %d\n", k, L); return 1; }
        dsv4_gpu_attn_cfg ac = {
            .hidden = c.hidden, .q_lora = c.q_lora, .n_heads = c.n_heads, .head_dim = hd,
            .rope_dim = c.qk_rope, .window = c.sliding_window, .ratio = ratio,
            .idx_heads = a->has_idx ? c.index_n_heads : 0, .idx_dim = c.index_head_dim,
            .idx_topk = c.index_topk, .o_groups = c.o_groups, .o_lora = c.o_lora,
            .max_pos = maxpos, .rms_eps = c.rms_eps};
        dsv4_gpu_attn_w aw = {
            .wq_a = a->wq_a, .wq_b = a->wq_b, .wkv = a->wkv, .wo_a = a->wo_a, .wo_b = a->wo_b,
            .q_norm = a->q_norm, .kv_norm = a->kv_norm, .sink = a->sink,
            .rope_cos = comp ? cs_c : cs_d, .rope_sin = comp ? sn_c : sn_d};
        if (a->has_comp) {
            aw.comp_wkv = a->comp.wkv; aw.comp_wgate = a->comp.wgate;
            aw.comp_norm = a->comp.norm; aw.comp_ape = a->comp.ape;
        }
        if (a->has_idx) { aw.idx_wq_b = a->idx.wq_b; aw.idx_wproj = a->idx.weights_proj; }
        if (dsv4_gpu_attn_bind(L, &ac, &aw) != 0) { fprintf(stderr, "attn: bind %d\n", L); return 1; }
        double worst = 0.0;
        for (int p = 0; p < n; p++) {
            if (dsv4_gpu_attn_step(got + (size_t)p * c.hidden,
                                   x + (size_t)L * per + (size_t)p * c.hidden, L, p) != 0) {
                fprintf(stderr, "attn: step layer %d pos %d failed\n", L, p);
                return 1;
            }
            const double r = vec_rel(got + (size_t)p * c.hidden,
                                     ref + (size_t)L * per + (size_t)p * c.hidden, c.hidden);
            printf("layer %d ratio %d pos %d rel %.3g\n", L, ratio, p, r);
            if (r > worst) worst = r;
            bad += !(r <= tol);
            steps++;
        }
        printf("layer %d ratio %d indexer %d: worst_rel %.3g over %d positions\n", L, ratio,
               a->has_idx, worst, n);
        if (worst > worst_all) worst_all = worst;
    }
    printf("summary: layers %d steps %d worst_rel %.3g over_tol %d tol %.3g\n", c.n_layers,
           steps, worst_all, bad, tol);
    dsv4_gpu_shutdown();
    return bad == 0 ? 0 : 1;
}
