"""End-to-end decode on the CPU (the harness half).

The tiny checkpoint written by tests/tiny_checkpoint.py is loaded by the
reference's own config reader, safetensors reader and binder. It is then
decoded by its own dsv4_layer_forward over 46 teacher-forced positions,
twice from fresh state. The two passes must agree bit for bit. This proves
the generator's schema and the driver before the GPU run compares the
MI355X trunk with this path (tests/test_gpu_e2e.py).
"""
import pytest

import e2e_common

pytestmark = pytest.mark.skipif(not e2e_common.available(),
                                reason="oracle/_ref/dsv4_e2e not built (needs /root/reference)")


def test_reference_decode_runs_and_is_deterministic(tmp_path):
    ckpt, tf = e2e_common.prepare(tmp_path)
    p, rows, summ = e2e_common.run(ckpt, tf, cpu_only=True)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert summ and int(summ.group(1)) == 46 and int(summ.group(2)) == 46
    assert len(rows) == 46 and all(r["rel"] == 0.0 for r in rows)
    # the tokens really move the model: not one argmax everywhere
    assert len({r["ref"] for r in rows}) > 10


def test_reference_prefill_protocol_on_cpu(tmp_path):
    """The reference's batched prefill protocol (test_model_oracle.c:295-378)
    on the CPU: dsv4_layer_forward_n at chunks 1, 2, 3 and 46 gives logits
    bit-identical to the per-token decode. The GPU run repeats it with the
    device's batched matmuls (tests/test_gpu_e2e.py)."""
    ckpt, tf = e2e_common.prepare(tmp_path)
    p, rows, summ = e2e_common.run(ckpt, tf, cpu_only=True)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    s = p.summary45
    assert s, p.stdout[-2000:]
    assert s.group(1) == "1,2,3,46" and int(s.group(2)) == 4 * 46
    assert int(s.group(3)) == int(s.group(4)) == 4 * 46


def test_attention_driver_reference_pass(tmp_path):
    """oracle/_ref/dsv4_attn's first pass -- the reference's own attention()
    on every layer of the tiny checkpoint, called through the #included
    dsv4_layer.c -- runs to the end on the CPU (exit 2: no device for the
    second pass here; 0 where a device is present)."""
    import os
    import subprocess
    import tiny_checkpoint
    exe = os.path.join(e2e_common.ROOT, "oracle", "_ref", "dsv4_attn")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/dsv4_attn not built")
    tiny_checkpoint.write(str(tmp_path))
    p = subprocess.run([exe, str(tmp_path), "12"], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode in (0, 2), p.stdout[-2000:] + p.stderr[-2000:]
    assert "attention: 1 dense + 2 indexed(top3) + 1 compressed(1:8)" in p.stdout + p.stderr
