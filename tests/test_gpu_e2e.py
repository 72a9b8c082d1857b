"""End-to-end greedy decode, GPU trunk against the CPU path (BASELINE
configs[4]): 46 teacher-forced random token ids in [0, 129280) through a tiny,
structurally real deepseek_v4 checkpoint (FP8 trunk, MXFP4 experts, CSA
indexer with selection, sparse MLA), run by the reference's own C99 model
code. In the second pass every FP8 matrix the reference uploads
(dsv4_run.c:270-283) runs on the MI355X through dsv4_gpu_mmq. That includes
the wo_a group slices, which resolve as row-range views. Every expert's FP4
matrices and every BF16 matrix (router gates, compressors, indexer weights, the
LM head) are resident too (they run on the device through the same dispatch),
and attention()'s CSA calls -- indexer score, top-k, sparse
attention (dsv4_layer.c:286-301) -- go to dsv4_gpu_indexer_score /
dsv4_gpu_topk / dsv4_gpu_sparse_attn.

A third pass takes every layer's attention() output from the device
attention block instead (dsv4_gpu_attn_step, one call per layer and
position), and its routed experts' k-ordered sum from the fused pass
(dsv4_gpu_moe_fp4) (oracle/e2e_decode.c, e2e_mmq).

Bar: identical argmax at every position, in both GPU passes. The logits
agree within the reference's own whole-model tolerance, 2e-3 vector-scaled
(tests/unit/test_model_oracle.c:253-270).
"""
import sys

import pytest

import e2e_common

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not e2e_common.available(),
                                 reason="oracle/_ref/dsv4_e2e not built")]


def test_gpu_trunk_argmax_identical(tmp_path):
    ckpt, tf = e2e_common.prepare(tmp_path)
    print("e2e: checkpoint %s, running the GPU trunk pass" % ckpt, flush=True)
    p, rows, summ = e2e_common.run(ckpt, tf)
    print(p.stdout[-4000:], flush=True)
    sys.stdout.flush()
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert summ, p.stdout[-2000:]
    n, agree, worst, mats = (int(summ.group(1)), int(summ.group(2)),
                             float(summ.group(3)), int(summ.group(4)))
    fp4, score, topk, attn = (int(summ.group(i)) for i in range(5, 9))
    assert n == 46 and agree == 46
    assert mats >= 4 * 8            # every layer's FP8 trunk is resident
    assert fp4 >= 4 * 16 * 3        # every routed expert's w1, w2, w3
    assert attn == 46 * 4           # one sparse attention per layer and position
    assert score > 0 and topk == score   # the CSA layers selected on the device
    assert int(summ.group(9)) >= 1 + 4      # the LM head and every router gate
    assert int(summ.group(10)) == int(summ.group(11)) == 46   # dsv4_gpu_head_argmax
    assert worst < 2e-3
    assert any(r["rel"] > 0.0 for r in rows), "GPU pass produced CPU bits: trunk not on GPU?"
    # pass 3: every layer's attention() output from the device attention block
    s3 = p.summary3
    assert s3, p.stdout[-2000:]
    assert int(s3.group(1)) == 46 * 4 and int(s3.group(2)) == 46
    assert float(s3.group(3)) < 2e-3
    assert int(s3.group(4)) == 46 * 4          # every layer's routed experts fused
