"""Write tests/golden/reference_fixtures.json from the reference's own test fixtures.

Reads the safetensors data files under the reference's
crates/ltx-weights/tests/fixtures/ as plain bytes (header JSON + raw data;
nothing is executed or unpickled) and records the inputs and expected
outputs the reference's parity tests use (crates/ltx-weights/tests/parity.rs:23-75):

  fp8_e4m3fn_parity  : "w" F8_E4M3 [4,4] + "w_scale" F32 scalar
  fp8_e4m3fn_expected: "w" F32 [4,4]
  lora_parity_base   : "layer.weight" BF16 [8,4]
  lora_parity_lora   : "layer.lora_A.weight" F32 [2,4], "layer.lora_B.weight" F32 [8,2], "layer.alpha" F32
  lora_parity_expected: "layer.weight" BF16 [8,4] (merged at strength 0.75)

Usage: python tests/golden/extract_reference_fixtures.py [reference_root]
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import st_io  # noqa: E402

FIXTURES = "crates/ltx-weights/tests/fixtures"
FILES = [
    "fp8_e4m3fn_parity",
    "fp8_e4m3fn_expected",
    "lora_parity_base",
    "lora_parity_lora",
    "lora_parity_expected",
]


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = {"source": FIXTURES, "files": {}}
    for stem in FILES:
        tensors, meta = st_io.read(os.path.join(root, FIXTURES, stem + ".safetensors"))
        entry = {"metadata": meta, "tensors": {}}
        for name, (dtype, shape, arr) in sorted(tensors.items()):
            entry["tensors"][name] = {
                "dtype": dtype,
                "shape": shape,
                # raw little-endian payload, so every bit (NaN payloads, -0) survives
                "hex": arr.tobytes().hex(),
            }
        out["files"][stem] = entry
    with open(os.path.join(HERE, "reference_fixtures.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
