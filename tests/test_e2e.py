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
