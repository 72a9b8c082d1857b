"""The attention block on the device (dsv4_gpu_attn_step) against the
reference's own attention() (dsv4_layer.c:213-336), run by
oracle/_ref/dsv4_attn on the tiny checkpoint: every layer (compress ratio 0,
4 with the CSA indexer, 8), 40 positions from fresh state, each with its own
seeded input. The reference pass runs every matmul on its CPU path; the
device pass runs the whole block in one call per position.

Bar: every step within 1e-5 vector-scaled relative error, the attention
bar (measured: 1.2e-6 at worst). The block's GEMVs accumulate in fp32 where
the reference accumulates in double, and the block chains five of them, two
norms and the softmax.
"""
import os
import re
import subprocess
import sys

import pytest

import e2e_common
import tiny_checkpoint

ATTN = os.path.join(e2e_common.ROOT, "oracle", "_ref", "dsv4_attn")

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(ATTN),
                                 reason="oracle/_ref/dsv4_attn not built")]


def test_attention_block_matches_reference(tmp_path):
    tiny_checkpoint.write(str(tmp_path))
    print("attn: checkpoint %s" % tmp_path, flush=True)
    p = subprocess.run([ATTN, str(tmp_path), "40", "--tol", "1e-5"], capture_output=True,
                       text=True, timeout=300)
    print("\n".join(l for l in p.stdout.splitlines() if "worst" in l or "summary" in l),
          flush=True)
    sys.stdout.flush()
    m = re.search(r"summary: layers (\d+) steps (\d+) worst_rel (\S+) over_tol (\d+)",
                  p.stdout)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert m and int(m.group(1)) == 4 and int(m.group(2)) == 160 and int(m.group(4)) == 0
    per = re.findall(r"layer (\d+) ratio (\d+) indexer (\d+): worst_rel (\S+)", p.stdout)
    assert sorted({int(r) for _, r, _, _ in per}) == [0, 4, 8]
    assert any(int(i) for _, _, i, _ in per)          # a CSA layer selected on the device
    rels = [float(x) for x in re.findall(r"pos \d+ rel (\S+)", p.stdout)]
    assert len(rels) == 160 and max(rels) > 0.0       # the device really computed it


def test_attention_block_past_4096_compressed_rows(tmp_path):
    """16,600 positions on the tiny checkpoint: its ratio-4 layers reach 4,150
    compressed rows, past the 4,096 scores the one-launch top-k ranks, so the
    block's CSA selection runs the radix path (the score kernel's level-1
    histogram, then the partition and final passes); the ratio-8 layer
    attends to 2,075 compressed rows. Every step against the reference's
    attention(), bar 1e-5."""
    tiny_checkpoint.write(str(tmp_path))
    print("attn long: 16600 positions, checkpoint %s" % tmp_path, flush=True)
    p = subprocess.run([ATTN, str(tmp_path), "16600", "--tol", "1e-5"], capture_output=True,
                       text=True, timeout=600)
    print("\n".join(l for l in p.stdout.splitlines() if "worst" in l or "summary" in l),
          flush=True)
    sys.stdout.flush()
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    m = re.search(r"summary: layers (\d+) steps (\d+) worst_rel (\S+) over_tol (\d+)",
                  p.stdout)
    assert m and int(m.group(1)) == 4 and int(m.group(2)) == 66400 and int(m.group(4)) == 0
    per = re.findall(r"layer (\d+) ratio (\d+) indexer (\d+): worst_rel", p.stdout)
    assert sum(int(r) == 4 and int(i) for _, r, i in per) == 2   # both CSA layers selected


@pytest.mark.parametrize("n,ratio,topk", [(24, 4, 512), (40, 4, 4), (132, 128, 512),
                                          (20, 0, 512)])
def test_attention_block_flash_shapes(n, ratio, topk):
    """The same comparison at the DeepSeek-V4-Flash attention shapes (hidden
    4096, 64 heads x 512, q_lora 1024, wo_a 8 x 1024, window 128, indexer 64
    x 128), synthetic weights, one layer of each compress ratio; at 132
    positions the ratio-128 compressor has closed one window, so the last
    positions attend to a compressed row. With index_topk 512 the ratio-4
    layer's few compressed rows are all taken (the block skips the indexer);
    with index_topk 4 the indexer selects 4 of up to 10 rows on the device."""
    print("attn flash: %d positions, ratio %d, index_topk %d" % (n, ratio, topk), flush=True)
    p = subprocess.run([ATTN, "--flash", str(n), str(ratio), "--tol", "1e-5",
                        "--topk", str(topk)],
                       capture_output=True, text=True, timeout=300)
    line = [l for l in p.stdout.splitlines() if l.startswith("flash:")]
    print(line, flush=True)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    m = re.search(r"flash: ratio (\d+) positions (\d+) worst_rel (\S+) over_tol (\d+)",
                  p.stdout)
    assert m and int(m.group(2)) == n and int(m.group(4)) == 0
    rels = [float(x) for x in re.findall(r"flash pos \d+ rel (\S+)", p.stdout)]
    assert len(rels) == n and max(rels) > 0.0
