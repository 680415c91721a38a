"""Write tests/golden/tiny_qwen3_v2.smodel (and the _q8 and v1 variants) with the reference packer.

Builds a tiny seeded Qwen3-shaped Hugging Face checkpoint (config.json and
one fp32 SafeTensors file: 2 layers, hidden 128, 2 query heads and 1 KV head
of dim 64, FFN 256, vocab 256) in a temporary directory, then runs the
reference's stdlib-only packer (tools/silicatepack.py of silicatetech/zero,
read from /root/reference in the build container) as

    silicatepack pack-hf --quant auto --interleave 4 --payload-alignment 4096

which emits a `.smodel`-v2 native container: Q4_0X4 layer linears, Q8_0
token embedding, Q8_0X4 output.weight, F32 norms (silicatepack.py:799-852,
943-1059, 1097-1161).  The packer's own `inspect` record of that file
(header and manifest, silicatepack.py:1754-1780) is written next to it as
tiny_qwen3_v2.inspect.json.  The `_q8` variant packs a one-layer model of
the same shape with `--quant q8_0` (Q8_0X4 layer linears); the `v1` variant
packs a one-layer model with the packer's default layout (no --interleave:
a `.smodel`-v1 container of plain row-major Q4_0 linears and a plain Q8_0
output.weight, silicatepack.py:1434-1450).

These files are what travels; the reference and the SafeTensors input do
not.  Usage: python tests/golden/make_smodel_fixture.py [/path/to/reference]
[variant ...] (default: every variant)
"""
from __future__ import annotations

import json
import shutil
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# variant -> (file stem, packer --quant, layers, packer --interleave)
VARIANTS = {"auto": ("tiny_qwen3_v2", "auto", 2, 4), "q8_0": ("tiny_qwen3_v2_q8", "q8_0", 1, 4),
            "v1": ("tiny_qwen3_v1", "auto", 1, 0)}

CONFIG = {
    "model_type": "qwen3",
    "architectures": ["Qwen3ForCausalLM"],
    "hidden_size": 128,
    "intermediate_size": 256,
    "num_hidden_layers": 2,
    "num_attention_heads": 2,
    "num_key_value_heads": 1,
    "head_dim": 64,
    "vocab_size": 256,
    "max_position_embeddings": 64,
    "rope_theta": 1000000.0,
    "rms_norm_eps": 1e-6,
    "eos_token_id": 7,
}


def config(variant: str = "auto") -> dict:
    return dict(CONFIG, num_hidden_layers=VARIANTS[variant][2])


def checkpoint(seed: int = 20241, variant: str = "auto") -> dict[str, np.ndarray]:
    """Seeded fp32 weights with Hugging Face Qwen3 names."""
    rng = np.random.default_rng(seed)
    c = config(variant)
    h, f, v = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    hd = c["head_dim"]
    qd, kvd = c["num_attention_heads"] * hd, c["num_key_value_heads"] * hd

    def mat(rows, cols, scale):
        return (rng.standard_normal((rows, cols)) * scale).astype(np.float32)

    def gain(n):
        return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)

    t = {"model.embed_tokens.weight": mat(v, h, 1.0), "lm_head.weight": mat(v, h, 0.05),
         "model.norm.weight": gain(h)}
    for i in range(c["num_hidden_layers"]):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = gain(h)
        t[p + "post_attention_layernorm.weight"] = gain(h)
        t[p + "self_attn.q_proj.weight"] = mat(qd, h, 0.08)
        t[p + "self_attn.k_proj.weight"] = mat(kvd, h, 0.08)
        t[p + "self_attn.v_proj.weight"] = mat(kvd, h, 0.08)
        t[p + "self_attn.o_proj.weight"] = mat(h, qd, 0.08)
        t[p + "self_attn.q_norm.weight"] = gain(hd)
        t[p + "self_attn.k_norm.weight"] = gain(hd)
        t[p + "mlp.gate_proj.weight"] = mat(f, h, 0.08)
        t[p + "mlp.up_proj.weight"] = mat(f, h, 0.08)
        t[p + "mlp.down_proj.weight"] = mat(h, f, 0.06)
    return t


def main(ref_root: str, only: list[str] | None = None) -> None:
    from safetensors.numpy import save_file

    sys.path.insert(0, str(Path(ref_root) / "tools"))
    import silicatepack  # noqa: E402  (reference packer, stdlib only)

    for variant, (stem, quant, _, il) in VARIANTS.items():
        if only and variant not in only:
            continue
        out_file, out_json = HERE / f"{stem}.smodel", HERE / f"{stem}.inspect.json"
        with tempfile.TemporaryDirectory() as tmp:
            src = Path(tmp) / "hf"
            src.mkdir()
            (src / "config.json").write_text(json.dumps(config(variant)))
            save_file(checkpoint(variant=variant), str(src / "model.safetensors"))
            out = Path(tmp) / "tiny.smodel"
            args = ["pack-hf", "--input-dir", str(src), "--output", str(out), "--quant", quant,
                    "--payload-alignment", "4096", "--force"]
            if il:
                args += ["--interleave", str(il)]
            rc = silicatepack.main(args)
            if rc not in (0, None):
                raise SystemExit(f"packer failed: {rc}")
            record = silicatepack.inspect_path(out, json_output=False)
            record["file"] = out_file.name
            shutil.copyfile(out, out_file)
        out_json.write_text(json.dumps(record, indent=1, sort_keys=True) + "\n")
        print(f"wrote {out_file} ({out_file.stat().st_size} bytes) and {out_json}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", sys.argv[2:])
