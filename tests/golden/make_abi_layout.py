"""Writes tests/golden/abi_layout.json: sizes, field offsets and constants of
the reference ABI header (c/cuda/qwn_cuda_abi.h), read in place under
/root/reference.  Run once in the build container; the JSON is the fixture."""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from abi_layout_probe import probe  # noqa: E402

REF_HEADER = "/root/reference/c/cuda/qwn_cuda_abi.h"

if __name__ == "__main__":
    layout = probe(REF_HEADER)
    layout["source"] = "c/cuda/qwn_cuda_abi.h"
    with open(os.path.join(HERE, "abi_layout.json"), "w") as f:
        json.dump(layout, f, indent=1, sort_keys=True)
    print("wrote abi_layout.json")
