"""Writes the manifest fixtures under tests/golden/manifests/ from the reference's own data files (JSON IO tables and a
.layout text file: data, no code). Run in a container that holds the reference:

    python tests/golden/make_manifest_fixtures.py /root/reference

Kept per manifest: format, model, context, cores, params, and the kernels of the roles the axk tests bind (the decode
group, the output head, the 35B's packed and plain prefill layer kernels and one MoE slots kernel); the ViT and the
other prefill variants are dropped.
"""
import json
import os
import shutil
import sys

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "manifests")
SOURCES = {
    "qwen35_9b_c131072.manifest.json": ("models/qwen35_9b/whole/qwen35_9b_c131072.manifest.json",
                                        ("decode.group", "lm_head")),
    "qwen35_35b_a3b.manifest.json": ("models/qwen35_35b_a3b/qwen35_35b_a3b.manifest.json",
                                     ("decode.group", "lm_head", "prefill256.gdn", "prefill256.attn", "prefill64.gdn",
                                      "prefill64.attn", "moe.slots32_g64")),
}
LAYOUTS = {"qwen35_9b_group16_gggagggagggaggga_mx4_kvc_c16384_npu4.layout":
           "models/qwen35_9b/whole/kernels/qwen35_9b_group16_gggagggagggaggga_mx4_kvc_c16384_npu4.layout"}


def main(ref: str) -> None:
    os.makedirs(HERE, exist_ok=True)
    for out, (src, roles) in SOURCES.items():
        m = json.load(open(os.path.join(ref, src)))
        keep = {k: m[k] for k in ("format", "model", "context", "cores", "params")}
        keep["kernels"] = {r: m["kernels"][r] for r in roles}
        with open(os.path.join(HERE, out), "w") as f:
            json.dump(keep, f, indent=0, separators=(",", ":"))
            f.write("\n")
    for out, src in LAYOUTS.items():
        shutil.copyfile(os.path.join(ref, src), os.path.join(HERE, out))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
