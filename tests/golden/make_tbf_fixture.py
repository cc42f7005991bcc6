"""Write tiny .tbf files with the reference converter's own TBF writer.

Runs ONLY in the build container, where the reference tree is mounted: it
imports ``write_tbf_format`` and ``ModelConfig`` from
``Scripts/convert_model.py`` (vivekptnk/tinybrain; writer at lines 462-706,
header at 48-70) and writes a one-layer LLaMA-shaped model from seeded
float32 weights, once with INT8 per-channel and once with INT4 group-32
quantization.  Only the written files and the float32 source arrays are
kept (beside this script); the reference source is not copied.

    python tests/golden/make_tbf_fixture.py [/root/reference]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DIMS = dict(num_layers=1, hidden_dim=32, num_heads=2, num_kv_heads=1, intermediate_dim=64,
            vocab_size=40, max_seq_len=64)


def source_weights():
    rng = np.random.default_rng(20250602)
    H, I, V = DIMS["hidden_dim"], DIMS["intermediate_dim"], DIMS["vocab_size"]
    kv = H // DIMS["num_heads"] * DIMS["num_kv_heads"]
    f = lambda *s: rng.normal(0.0, 0.02, size=s).astype(np.float32)
    norm = lambda: (1.0 + 0.1 * rng.normal(size=H)).astype(np.float32)
    layer = {"q_proj": f(H, H), "k_proj": f(kv, H), "v_proj": f(kv, H), "o_proj": f(H, H),
             "gate_proj": f(I, H), "up_proj": f(I, H), "down_proj": f(H, I),
             "input_layernorm": norm(), "post_attention_layernorm": norm()}
    return {"embeddings": rng.normal(0.0, 1.0, size=(V, H)).astype(np.float32),
            "layers": [layer], "final_norm": norm(), "lm_head": f(V, H)}


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, os.path.join(ref, "Scripts"))
    from convert_model import ModelConfig, write_tbf_format  # reference converter

    w = source_weights()
    cfg = ModelConfig(**DIMS)
    write_tbf_format(w, cfg, os.path.join(HERE, "converter_tiny_int8.tbf"), quantize_mode="int8")
    write_tbf_format(w, cfg, os.path.join(HERE, "converter_tiny_int4.tbf"), quantize_mode="int4",
                     group_size=32)
    flat = {"embeddings": w["embeddings"], "final_norm": w["final_norm"], "lm_head": w["lm_head"]}
    for k, v in w["layers"][0].items():
        flat["layer0_" + k] = v
    np.savez(os.path.join(HERE, "converter_tiny_weights.npz"), **flat)


if __name__ == "__main__":
    main()
