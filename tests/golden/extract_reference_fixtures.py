"""Writes tests/golden/q5_k_gguf_py_block.json from the reference's own test data.

Run once in the build container (it reads /root/reference as text; nothing is
imported or executed from it).  The fixture is data: 176 raw bytes of a real
Q5_K super-block, 24 spot values and the 256-element sum that llama.cpp's
gguf-py produced for it (crates/ggml-cpu/src/dequant.rs:472-548).
"""
import json
import os
import re

SRC = "/root/reference/crates/ggml-cpu/src/dequant.rs"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q5_k_gguf_py_block.json")


def main() -> None:
    src = open(SRC).read()
    raw = re.search(r"const RAW: \[u8; 176\] = \[(.*?)\];", src, re.S).group(1)
    raw = [int(v) for v in raw.replace("\n", " ").split(",") if v.strip()]
    spots = re.search(r"const SPOTS: \[\(usize, f32\); 24\] = \[(.*?)\];", src, re.S).group(1)
    spots = [(int(a), float(b)) for a, b in re.findall(r"\((\d+),\s*([-0-9.e]+)\)", spots)]
    total = float(re.search(r"const SOMA: f64 = ([-0-9.e]+);", src).group(1))
    assert len(raw) == 176 and len(spots) == 24
    json.dump({"source": "crates/ggml-cpu/src/dequant.rs:472-548 (first Q5_K super-block of "
                         "Qwen2.5-32B-Instruct-Q5_K_M token_embd, values from llama.cpp gguf-py)",
               "type": 13, "raw": raw, "spots": spots, "sum": total,
               "spot_tol": 1e-6, "sum_tol": 1e-5}, open(OUT, "w"), indent=1)


if __name__ == "__main__":
    main()
