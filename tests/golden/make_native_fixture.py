"""Write ``tests/golden/native_fixture.npz`` from the reference's test fixture.

Reads the data files of ``test/fixtures/native/`` under ``/root/reference``
(config.json, model.safetensors, readout.safetensors, reference.json,
cuda_reference.json) with safe loaders only (JSON and safetensors) and stores
them as plain numpy arrays: the tiny random-init weights, the readout and, per
case, the token ids, masks and the expected PyTorch logits.  Run once in a
container that has the reference mounted; the npz is what tests load.
"""
import json
import os
import sys

import numpy as np
from safetensors.numpy import load_file

SRC = "/root/reference/test/fixtures/native"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native_fixture.npz")


def main():
    if not os.path.isdir(SRC):
        sys.exit(f"reference fixture not found at {SRC}")
    arrays = {}
    with open(os.path.join(SRC, "config.json")) as f:
        config = json.load(f)
    arrays["config_json"] = np.array(json.dumps(config))
    for name, value in load_file(os.path.join(SRC, "model.safetensors")).items():
        assert value.dtype == np.float32, (name, value.dtype)
        key = name[name.index("language_model."):][len("language_model."):]
        arrays["w/" + key] = value
    arrays["readout"] = load_file(os.path.join(SRC, "readout.safetensors"))["weight"]
    names = []
    for tag, fname in (("ref", "reference.json"), ("cuda", "cuda_reference.json")):
        with open(os.path.join(SRC, fname)) as f:
            cases = json.load(f)
        for i, case in enumerate(cases):
            label = f"{tag}{i:02d}"
            names.append(f"{label}:{case.get('name', '')}")
            arrays[f"case/{label}/ids"] = np.array(case["inputs"]["input_ids"], np.int32)
            arrays[f"case/{label}/mask"] = np.array(case["inputs"]["attention_mask"], np.int8)
            arrays[f"case/{label}/logits"] = np.array(case["logits"], np.float32)
    arrays["case_names"] = np.array(names)
    np.savez_compressed(DST, **arrays)
    print(f"wrote {DST}: {len(names)} cases, {sum(1 for k in arrays if k.startswith('w/'))} tensors")


if __name__ == "__main__":
    main()
