"""Helpers for the end-to-end decode test: write the
tiny checkpoint and token file, run oracle/_ref/dsv4_e2e, parse its report."""
import os
import re
import subprocess

import tiny_checkpoint

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E2E = os.path.join(ROOT, "oracle", "_ref", "dsv4_e2e")


def available():
    return os.path.exists(E2E)


def prepare(tmp_dir, n=46):
    tiny_checkpoint.write(str(tmp_dir))
    tok = tiny_checkpoint.tokens(n)
    tf = os.path.join(str(tmp_dir), "tokens.txt")
    with open(tf, "w") as f:
        f.write("\n".join(str(int(t)) for t in tok) + "\n")
    return str(tmp_dir), tf


def run(ckpt, tokens_file, cpu_only=False, timeout=300):
    cmd = [E2E, ckpt, tokens_file] + (["--cpu-only"] if cpu_only else [])
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    rows = []
    for line in p.stdout.splitlines():
        m = re.match(r"pos (\d+) tok (\d+) cpu (\d+) \w+ (\d+) margin (\S+) rel (\S+)", line)
        if m:
            rows.append(dict(pos=int(m.group(1)), tok=int(m.group(2)),
                             ref=int(m.group(3)), got=int(m.group(4)),
                             margin=float(m.group(5)), rel=float(m.group(6))))
    summ = re.search(r"summary: positions (\d+) argmax_equal (\d+) worst_rel (\S+) "
                     r"gpu_mats (\d+) fp4_mats (\d+) gpu_score (\d+) gpu_topk (\d+) "
                     r"gpu_attn (\d+) bf16_mats (\d+) head_ok (\d+)/(\d+)", p.stdout)
    p.summary3 = re.search(r"summary3: attention blocks on the device: steps (\d+) "
                           r"argmax_equal (\d+) worst_rel (\S+) fused_moe (\d+)", p.stdout)
    p.summary45 = re.search(r"summary45: prefill chunks (\S+) positions (\d+) "
                            r"pass4_bit_identical (\d+) pass4_argmax_equal (\d+) "
                            r"pass5_bit_identical (\d+) pass5_argmax_equal (\d+) "
                            r"moe_n_calls (\d+)", p.stdout)
    p.load = re.search(r"load: (\d+) shards, (\d+) tensors indexed; (\d+) matrices and "
                       r"(\d+) experts read into HBM, (\d+) bytes in (\S+) s \((\S+) GB/s\)",
                       p.stdout)
    return p, rows, summ
