/* SPDX-License-Identifier: Apache-2.0 */
/* moe_ref.c - the reference's own moe() (src/model/dsv4_layer.c:369-484),
 * callable from the checker, to pin the oracle's routed-expert sum.
 *
 * TEST INFRASTRUCTURE ONLY. moe() is static in the reference, so this file
 * #includes dsv4_layer.c as it lies under /root/reference and calls it;
 * oracle/Makefile compiles it with the reference's core sources into
 * oracle/_ref/libdsv4moe.so, whose only export is ref_moe_routed. The
 * matmul dispatch's device branch (dsv4_matmul.c:525) resolves against the
 * backend's CPU stub (deepseek-v4-in-c_amd/lib/libdsv4_gpu_stub.so), which
 * reports nothing resident, so every matmul runs on the reference's CPU
 * path. Nothing of the reference is copied.
 *
 * One call: a layer with n_exp FP4 routed experts (1x32 E8M0 blocks, the
 * expert cache's layout), a BF16 router gate, hash routing (tid2eid) so the
 * caller chooses the experts of token 0, and a shared expert of zeros, so
 * moe()'s output is its routed k-ordered sum (dsv4_layer.c:471-475) with
 * an exact +0.0 added per element. The router's weights come from the gate
 * as the model computes them (dsv4_route, dsv4_ops.c:103-136); idx_out and
 * w_out return the selection and weights moe() used.
 */
#include "dsv4_layer.c"

typedef struct {
    DSV4ExpertW *e;
    int n;
} MoeRefExperts;

static const DSV4ExpertW *moe_ref_get(void *ctx, int layer, int expert)
{
    const MoeRefExperts *E = ctx;
    (void)layer;
    return expert >= 0 && expert < E->n ? &E->e[expert] : NULL;
}

static DSV4QMat moe_ref_qmat(const void *w, const void *s, int wdt, int rows, int cols)
{
    DSV4QMat m = {w, s, wdt, rows, cols, wdt == DSV4_WFP4 ? 1 : 0, wdt == DSV4_WFP4 ? 32 : 0};
    return m;
}

int ref_moe_routed(float *out, int *idx_out, float *w_out, const float *x, int hidden,
                   int inter, int n_exp, int topk, const uint8_t *const *w1,
                   const uint8_t *const *s1, const uint8_t *const *w3,
                   const uint8_t *const *s3, const uint8_t *const *w2,
                   const uint8_t *const *s2, const int64_t *ids, const uint16_t *gate,
                   float swiglu_limit, float routed_scale)
{
    if (hidden <= 0 || inter <= 0 || n_exp <= 0 || topk <= 0 || topk > DSV4_MAX_TOPK ||
        topk > n_exp)
        return -1;
    DSV4Cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = hidden;
    c.moe_inter = inter;
    c.n_experts = n_exp;
    c.topk = topk;
    c.n_shared = 1;
    c.swiglu_limit = swiglu_limit;
    c.routed_scale = routed_scale;

    DSV4ExpertW *ex = calloc((size_t)n_exp, sizeof *ex);
    uint16_t *zero = calloc((size_t)inter * hidden, sizeof(uint16_t));
    DSV4Scratch s;
    memset(&s, 0, sizeof s);
    s.gate_scores = calloc((size_t)n_exp, sizeof(float));
    s.gate_orig = calloc((size_t)n_exp, sizeof(float));
    s.expert_gate = calloc((size_t)inter, sizeof(float));
    s.expert_up = calloc((size_t)inter, sizeof(float));
    s.expert_out = calloc((size_t)inter, sizeof(float));
    s.expert_acc = calloc((size_t)topk * hidden, sizeof(float));
    s.expert_acc_stride = hidden;
    int rc = -1;
    if (!ex || !zero || !s.gate_scores || !s.gate_orig || !s.expert_gate || !s.expert_up ||
        !s.expert_out || !s.expert_acc)
        goto done;
    for (int e = 0; e < n_exp; e++) {
        ex[e].w1 = moe_ref_qmat(w1[e], s1[e], DSV4_WFP4, inter, hidden);
        ex[e].w3 = moe_ref_qmat(w3[e], s3[e], DSV4_WFP4, inter, hidden);
        ex[e].w2 = moe_ref_qmat(w2[e], s2[e], DSV4_WFP4, hidden, inter);
    }
    DSV4LayerW w;
    memset(&w, 0, sizeof w);
    w.moe.gate = moe_ref_qmat(gate, NULL, DSV4_WBF16, n_exp, hidden);
    w.moe.tid2eid = ids;
    w.moe.shared.w1 = moe_ref_qmat(zero, NULL, DSV4_WBF16, inter, hidden);
    w.moe.shared.w3 = moe_ref_qmat(zero, NULL, DSV4_WBF16, inter, hidden);
    w.moe.shared.w2 = moe_ref_qmat(zero, NULL, DSV4_WBF16, hidden, inter);
    w.hash_routed = 1;
    MoeRefExperts E = {ex, n_exp};
    DSV4ExpertSrc src;
    memset(&src, 0, sizeof src);
    src.get = moe_ref_get;
    src.ctx = &E;
    moe(out, x, &w, &c, &s, &src, 0, 0);
    for (int k = 0; k < topk; k++) {
        idx_out[k] = s.topk_idx[k];
        w_out[k] = s.topk_w[k];
    }
    rc = 0;
done:
    free(ex); free(zero);
    free(s.gate_scores); free(s.gate_orig); free(s.expert_gate); free(s.expert_up);
    free(s.expert_out); free(s.expert_acc);
    return rc;
}
