"""End-to-end greedy decode, GPU trunk against the CPU path (BASELINE
configs[4]): 46 teacher-forced random token ids in [0, 129280) through a tiny,
structurally real deepseek_v4 checkpoint (FP8 trunk, MXFP4 experts, CSA
indexer with selection, sparse MLA), run by the reference's own C99 model
code. Before the second pass the backend's loader reads the checkpoint
straight into HBM (dsv4_gpu_ckpt_load_layer / _load_qmat, no per-matrix host
upload): every FP8 trunk matrix, every BF16 matrix (router gates,
compressors, indexer weights, the LM head) and every routed expert. The
binder's matrices are swapped for the resident ones, so every matmul runs on
the MI355X through the reference's dispatch (dsv4_gpu_mmq), including the
wo_a group slices, which resolve as row-range views of a loaded matrix; and
attention()'s CSA calls -- indexer score, top-k, sparse
attention (dsv4_layer.c:286-301) -- go to dsv4_gpu_indexer_score /
dsv4_gpu_topk / dsv4_gpu_sparse_attn.

A third pass takes every layer's attention() output from the device
attention block instead (dsv4_gpu_attn_step, one call per layer and
position), and its routed experts' k-ordered sum from the fused pass
(dsv4_gpu_moe_fp4) (oracle/e2e_decode.c, e2e_mmq).

Passes 4 and 5 run the reference's batched prefill protocol
(tests/unit/test_model_oracle.c:295-378): dsv4_layer_forward_n at chunks 1,
2, 3 and 46 from fresh state. Pass 4 keeps pass 2's residency and device CSA
calls, so moe_n's batched matmuls (router gate, the batch's routed experts,
shared expert; dsv4_layer.c:714-855) run through dsv4_gpu_mmq_n; pass 5 adds
pass 3's attention block and takes moe_n's routed sum from
dsv4_gpu_moe_fp4_n. Each position's logits must be bit-identical to the
per-token GPU pass with the same device parts.

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
    # the checkpoint was read into HBM by the loader: 4 layers of 8 FP8 + 1
    # BF16 matrices, 2 compressor BF16 on the 3 compressed layers, 1 FP8 + 3
    # BF16 indexer matrices on the 2 CSA layers, the head; 4 x 16 experts
    ld = p.load
    assert ld, p.stdout[-2000:]
    print("load: %s matrices and %s experts, %s bytes in %s s (%s GB/s)"
          % (ld.group(3), ld.group(4), ld.group(5), ld.group(6), ld.group(7)), flush=True)
    assert int(ld.group(3)) == 4 * 9 + 3 * 2 + 2 * 4 + 1
    assert int(ld.group(4)) == 4 * 16
    assert int(ld.group(5)) > 0 and float(ld.group(6)) > 0.0
    # pass 3: every layer's attention() output from the device attention block
    s3 = p.summary3
    assert s3, p.stdout[-2000:]
    assert int(s3.group(1)) == 46 * 4 and int(s3.group(2)) == 46
    assert float(s3.group(3)) < 2e-3
    assert int(s3.group(4)) == 46 * 4          # every layer's routed experts fused
    # passes 4 and 5: the batched prefill, bit for bit against the per-token passes
    s45 = p.summary45
    assert s45, p.stdout[-2000:]
    print("prefill: chunks %s, pass 4 %s/%s bit-identical, pass 5 %s/%s, %s batched MoE calls"
          % (s45.group(1), s45.group(3), s45.group(2), s45.group(5), s45.group(2),
             s45.group(7)), flush=True)
    assert s45.group(1) == "1,2,3,46" and int(s45.group(2)) == 4 * 46
    assert int(s45.group(3)) == int(s45.group(4)) == 4 * 46
    assert int(s45.group(5)) == int(s45.group(6)) == 4 * 46
    # moe_n once per layer and chunk of every chunking: 46 + 23 + 16 + 1 chunks
    assert int(s45.group(7)) == 4 * (46 + 23 + 16 + 1)


def test_gpu_trunk_matrix_core_form(tmp_path, monkeypatch):
    """The same run with DSV4_GPU_FP8_MX=1: the FP8 trunk takes the bf16
    matrix-core form, one token at a time (k_fp8_mx1) in passes 2 and 3 and
    batched in passes 4 and 5 (chunks of 2 and 3 on the register-staged
    kernel, 23 and 46 tokens on the DMA-staged one; a kernel trace of this
    run lists k_fp8_mx1, k_fp8_mxn and k_fp8_mxd). The reference's prefill
    protocol must still give every position the per-token pass's bits, and
    the argmax must still match the CPU reference at every position."""
    monkeypatch.setenv("DSV4_GPU_FP8_MX", "1")
    ckpt, tf = e2e_common.prepare(tmp_path)
    print("e2e: checkpoint %s, matrix-core FP8 form" % ckpt, flush=True)
    p, rows, summ = e2e_common.run(ckpt, tf)
    print(p.stdout[-3000:], flush=True)
    sys.stdout.flush()
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert summ, p.stdout[-2000:]
    assert int(summ.group(1)) == 46 and int(summ.group(2)) == 46
    assert float(summ.group(3)) < 2e-3
    s45 = p.summary45
    assert s45, p.stdout[-2000:]
    assert s45.group(1) == "1,2,3,46" and int(s45.group(2)) == 4 * 46
    assert int(s45.group(3)) == int(s45.group(4)) == 4 * 46
    assert int(s45.group(5)) == int(s45.group(6)) == 4 * 46
