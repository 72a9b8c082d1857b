"""A tiny but structurally real deepseek_v4 checkpoint for the end-to-end test
written with numpy in the reference's own schema.

What it matches in the reference:
- the tensor names, shapes and dtypes its binder requests
  (src/model/dsv4_bind.c:152-256, the plan walked by dsv4_bind_layer);
- the strict config schema of include/dsv4/dsv4_cfg.h:112-406 (every field
  present, none defaulted);
- the safetensors container its reader parses (src/io/dsv4_st.c).

The field set follows the reference's tools/make_tiny_checkpoint.py:234-257.
The configuration differs where the end-to-end workload (BASELINE.json
configs[4]) asks it to:
- the vocabulary is 129280;
- FP8 block scales and FP4 block scales vary;
- the experts are MXFP4;
- the layers cover compress ratios {0, 4, 8};
- index_topk is below the number of compressed rows, so the indexer selects.

Every FP8/FP4 value is drawn from the set its format represents exactly, so
the stored byte IS the value.

Usage: python tests/tiny_checkpoint.py DIR   (or write(DIR, seed) from Python)
"""
import json
import os
import struct
import sys

import numpy as np

CFG = dict(hidden=128, n_layers=4, vocab=129280, hc_mult=2,
           n_heads=4, head_dim=64, qk_rope=16, q_lora=64,
           o_lora=32, o_groups=2, window=8,
           n_experts=16, topk=4, moe_inter=64, n_shared=1,
           route_scale=1.5, swiglu_limit=10.0,
           rms_eps=1e-6, hc_eps=1e-6, sinkhorn_iters=20,
           num_hash_layers=1,
           index_n_heads=8, index_head_dim=64, index_topk=3,
           compress_ratios=[0, 4, 8, 4, 0])   # 4 decoder layers + 1 MTP tail


def _e4m3(b):
    s = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 7
    if e == 15 and m == 7:
        return float("nan")
    return s * (m * 2.0 ** -9 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7))


# e4m3 codes with 0 < |v| <= 0.5: finite, exact, and small enough to keep
# the activations of a random network in range.
_E4M3_SMALL = np.array([b for b in range(256)
                        if not np.isnan(_e4m3(b)) and 0.0 < abs(_e4m3(b)) <= 0.5],
                       np.uint8)


def _bf16(a):
    """bf16 bit patterns of float32 values (round to nearest even)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16))


class _Writer:
    def __init__(self, rng):
        self.rng = rng
        self.t = {}

    def fp8(self, name, rows, cols, blk=128):
        codes = _E4M3_SMALL[self.rng.integers(0, _E4M3_SMALL.size, (rows, cols))]
        sr, sc = max(1, -(-rows // blk)), max(1, -(-cols // blk))
        scales = self.rng.integers(126, 129, (sr, sc)).astype(np.uint8)   # 2^-1..2^1
        self.t[name + ".weight"] = ("F8_E4M3", codes)
        self.t[name + ".scale"] = ("F8_E8M0", scales)

    def fp4(self, name, rows, cols, blk=32):
        codes = self.rng.integers(0, 16, (rows, cols)).astype(np.uint8)
        packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
        scales = self.rng.integers(125, 128, (rows, max(1, cols // blk))).astype(np.uint8)
        self.t[name + ".weight"] = ("I8", packed)
        self.t[name + ".scale"] = ("F8_E8M0", scales)

    def bf16(self, name, *shape, scale=0.1):
        v = self.rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
        self.t[name] = ("BF16", _bf16(v))

    def f32(self, name, *shape, scale=1.0, add=0.0):
        v = self.rng.standard_normal(shape).astype(np.float32) * np.float32(scale)
        self.t[name] = ("F32", (v + np.float32(add)).astype(np.float32))

    def i64(self, name, arr):
        self.t[name] = ("I64", np.ascontiguousarray(arr, np.int64))

    def save(self, path):
        hdr, off, blobs = {}, 0, []
        for name, (dt, a) in self.t.items():
            b = np.ascontiguousarray(a).tobytes()
            hdr[name] = {"dtype": dt, "shape": list(a.shape),
                         "data_offsets": [off, off + len(b)]}
            blobs.append(b)
            off += len(b)
        j = json.dumps(hdr, separators=(",", ":")).encode()
        j += b" " * ((-(8 + len(j))) % 8)
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(j)))
            f.write(j)
            for b in blobs:
                f.write(b)
        return 8 + len(j) + off


def config_json(c=CFG):
    return {
        "architectures": ["DeepseekV4ForCausalLM"], "model_type": "deepseek_v4",
        "hidden_size": c["hidden"], "num_hidden_layers": c["n_layers"],
        "vocab_size": c["vocab"], "rms_norm_eps": c["rms_eps"],
        "max_position_embeddings": 4096,
        "num_attention_heads": c["n_heads"], "num_key_value_heads": 1,
        "head_dim": c["head_dim"], "q_lora_rank": c["q_lora"],
        "o_lora_rank": c["o_lora"], "o_groups": c["o_groups"],
        "qk_rope_head_dim": c["qk_rope"], "sliding_window": c["window"],
        "index_n_heads": c["index_n_heads"], "index_head_dim": c["index_head_dim"],
        "index_topk": c["index_topk"], "compress_rope_theta": 160000.0,
        "compress_ratios": c["compress_ratios"],
        "hc_mult": c["hc_mult"], "hc_sinkhorn_iters": c["sinkhorn_iters"],
        "hc_eps": c["hc_eps"],
        "n_routed_experts": c["n_experts"], "num_experts_per_tok": c["topk"],
        "n_shared_experts": c["n_shared"], "moe_intermediate_size": c["moe_inter"],
        "routed_scaling_factor": c["route_scale"], "norm_topk_prob": True,
        "scoring_func": "sqrtsoftplus", "topk_method": "noaux_tc",
        "swiglu_limit": c["swiglu_limit"], "rope_theta": 10000.0,
        "rope_scaling": {"type": "yarn", "factor": 16, "beta_fast": 32,
                         "beta_slow": 1, "original_max_position_embeddings": 2048},
        "num_hash_layers": c["num_hash_layers"], "num_nextn_predict_layers": 1,
        "expert_dtype": "fp4", "torch_dtype": "bfloat16",
        "quantization_config": {"activation_scheme": "dynamic", "fmt": "e4m3",
                                "quant_method": "fp8", "scale_fmt": "ue8m0",
                                "weight_block_size": [128, 128]},
    }


def write(out_dir, seed=4242, c=CFG):
    """Write config.json and one safetensors shard into out_dir; returns the
    shard's byte count."""
    os.makedirs(out_dir, exist_ok=True)
    rng = np.random.default_rng(seed)
    W = _Writer(rng)
    H, hd, d = c["n_heads"], c["head_dim"], c["hidden"]
    hc = c["hc_mult"]
    mix = (2 + hc) * hc
    W.bf16("embed.weight", c["vocab"], d, scale=0.5)
    W.f32("norm.weight", d, scale=0.1, add=1.0)
    W.bf16("head.weight", c["vocab"], d, scale=0.3)
    W.f32("hc_head_fn", hc, hc * d, scale=0.05)
    W.f32("hc_head_base", hc, scale=0.3)
    W.f32("hc_head_scale", 1, scale=0.1, add=1.0)
    for L in range(c["n_layers"]):
        ratio = c["compress_ratios"][L]
        coff = 2 if ratio == 4 else 1
        p = "layers.%d" % L
        W.f32(p + ".attn_norm.weight", d, scale=0.1, add=1.0)
        W.f32(p + ".ffn_norm.weight", d, scale=0.1, add=1.0)
        W.f32(p + ".attn.attn_sink", H, scale=1.0)
        W.f32(p + ".attn.q_norm.weight", c["q_lora"], scale=0.1, add=1.0)
        W.f32(p + ".attn.kv_norm.weight", hd, scale=0.1, add=1.0)
        W.fp8(p + ".attn.wq_a", c["q_lora"], d)
        W.fp8(p + ".attn.wq_b", H * hd, c["q_lora"])
        W.fp8(p + ".attn.wkv", hd, d)
        W.fp8(p + ".attn.wo_a", c["o_groups"] * c["o_lora"], H * hd // c["o_groups"])
        W.fp8(p + ".attn.wo_b", d, c["o_groups"] * c["o_lora"])
        if ratio:
            W.f32(p + ".attn.compressor.ape", ratio, coff * hd, scale=0.5)
            W.f32(p + ".attn.compressor.norm.weight", hd, scale=0.1, add=1.0)
            W.bf16(p + ".attn.compressor.wkv.weight", coff * hd, d)
            W.bf16(p + ".attn.compressor.wgate.weight", coff * hd, d)
        if ratio == 4:
            ih, idd = c["index_n_heads"], c["index_head_dim"]
            W.fp8(p + ".attn.indexer.wq_b", ih * idd, c["q_lora"])
            W.bf16(p + ".attn.indexer.weights_proj.weight", ih, d)
            W.f32(p + ".attn.indexer.compressor.ape", ratio, 2 * idd, scale=0.5)
            W.f32(p + ".attn.indexer.compressor.norm.weight", idd, scale=0.1, add=1.0)
            W.bf16(p + ".attn.indexer.compressor.wkv.weight", 2 * idd, d)
            W.bf16(p + ".attn.indexer.compressor.wgate.weight", 2 * idd, d)
        W.f32(p + ".hc_attn_fn", mix, hc * d, scale=0.05)
        W.f32(p + ".hc_ffn_fn", mix, hc * d, scale=0.05)
        W.f32(p + ".hc_attn_base", mix, scale=0.3)
        W.f32(p + ".hc_ffn_base", mix, scale=0.3)
        W.f32(p + ".hc_attn_scale", 3, scale=0.1, add=1.0)
        W.f32(p + ".hc_ffn_scale", 3, scale=0.1, add=1.0)
        W.bf16(p + ".ffn.gate.weight", c["n_experts"], d, scale=0.3)
        if L < c["num_hash_layers"]:
            # topk DISTINCT experts per token, as hash routing gives them: the
            # batched prefill relies on it (dsv4_layer.c:670-676, a token is
            # routed to an expert at most once)
            W.i64(p + ".ffn.gate.tid2eid",
                  np.argsort(rng.random((c["vocab"], c["n_experts"])), axis=1)[:, :c["topk"]])
        else:
            W.f32(p + ".ffn.gate.bias", c["n_experts"], scale=0.5)
        for e in range(c["n_experts"]):
            W.fp4("%s.ffn.experts.%d.w1" % (p, e), c["moe_inter"], d)
            W.fp4("%s.ffn.experts.%d.w2" % (p, e), d, c["moe_inter"])
            W.fp4("%s.ffn.experts.%d.w3" % (p, e), c["moe_inter"], d)
        W.fp8(p + ".ffn.shared_experts.w1", c["moe_inter"] * c["n_shared"], d)
        W.fp8(p + ".ffn.shared_experts.w2", d, c["moe_inter"] * c["n_shared"])
        W.fp8(p + ".ffn.shared_experts.w3", c["moe_inter"] * c["n_shared"], d)
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(config_json(c), f, indent=2)
        f.write("\n")
    return W.save(os.path.join(out_dir, "model-00001-of-00001.safetensors"))


def tokens(n=46, seed=46, vocab=CFG["vocab"]):
    """n teacher-forced token ids drawn uniformly from [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int64)


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else "tiny_dsv4"
    n = write(out)
    print("%s: %d bytes" % (out, n))
