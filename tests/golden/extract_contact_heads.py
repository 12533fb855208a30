"""Writes codon-infer_amd/codon_hip/data/contact_heads.json: the ESM-2
contact-head logistic-regression weights (L*H weights, l-major, plus one bias
per architecture) as data.  An offline generator run once in the build
container; the package only reads the JSON it wrote.

Source: the `CONTACT_HEAD_*_WEIGHT` / `CONTACT_HEAD_*_BIAS` constant tables of
codon-infer's src/contact_heads.rs (lines 5, 24, 58, 137, 224), which hold
Meta's `esm.contact_head.regression` parameters.  The file is parsed as text;
nothing is executed.  Usage:
    python tests/golden/extract_contact_heads.py /path/to/codon-infer/src/contact_heads.rs
"""
import json
import os
import re
import sys

ARCHS = ["8M", "35M", "150M", "650M", "3B"]


def parse(text):
    out = {}
    for arch in ARCHS:
        b = re.search(rf"CONTACT_HEAD_{arch}_BIAS\s*:\s*f32\s*=\s*([-+0-9.eE]+)_f32", text)
        w = re.search(rf"CONTACT_HEAD_{arch}_WEIGHT\s*:\s*\[f32;\s*(\d+)\]\s*=\s*\[(.*?)\];", text, re.S)
        if not (b and w):
            raise ValueError(f"tables for {arch} not found")
        vals = [float(v) for v in re.findall(r"([-+0-9.eE]+)_f32", w.group(2))]
        if len(vals) != int(w.group(1)):
            raise ValueError(f"{arch}: {len(vals)} values, expected {w.group(1)}")
        out[arch] = {"bias": float(b.group(1)), "weight": vals}
    return out


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/contact_heads.rs"
    with open(src) as f:
        data = parse(f.read())
    repo = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    dst = os.path.join(repo, "codon-infer_amd", "codon_hip", "data", "contact_heads.json")
    with open(dst, "w") as f:
        json.dump(data, f)
    print("wrote", dst, {k: len(v["weight"]) for k, v in data.items()})


if __name__ == "__main__":
    main()
