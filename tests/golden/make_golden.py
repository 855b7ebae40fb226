"""Regenerate the committed golden fixtures under tests/golden/ from the reference checkout.

    python tests/golden/make_golden.py [/root/reference]

What it writes (all data, no code):

* `tiny-clf.tirs`, `tiny-reg.tirs`: the reference's tiny random-init TabICL v2 checkpoints
  (`tests/data/tiny-{clf,reg}.ckpt`, made by the reference's `tools/make_tiny.py`, seed 1 per
  `CONTRIBUTING.md:78-80`) converted to `.tirs` weight bundles. The checkpoints are PyTorch zip files; they are
  read with `torch.load(weights_only=True)`, which executes nothing from the file. Tensor names are the state-dict
  names (what the reference's own converter `src/ckpt.rs:299-339` writes), float32 throughout, plus a
  `config.json` uint8 tensor holding the checkpoint's config as JSON.
* `tiny-raw.tirs`, `tiny-one.tirs`, `tiny-table.tirs`, `tiny-many.tirs`, `tiny-reg-a.tirs`, `tiny-reg-b.tirs`:
  copied byte for byte from the reference's `tests/data/` (numbers dumped from upstream PyTorch TabICL by the
  reference's `tools/dump_raw.py`, `dump_table.py`, `dump_reg.py`).

The reference's licence (BSD 3-Clause) travels with them in `LICENSE-reference.txt`.
"""
import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def main(ref: str) -> None:
    import importlib

    import torch

    bundle = importlib.import_module("tabicl-anywhere_amd.bundle")
    data = os.path.join(ref, "tests", "data")
    for kind in ("clf", "reg"):
        ck = torch.load(os.path.join(data, f"tiny-{kind}.ckpt"), map_location="cpu", weights_only=True)
        tensors = {}
        for name, t in ck["state_dict"].items():
            tensors[name] = t.detach().to(torch.float32).contiguous().numpy()
        tensors["config.json"] = np.frombuffer(json.dumps(ck["config"]).encode(), dtype=np.uint8)
        out = os.path.join(HERE, f"tiny-{kind}.tirs")
        bundle.write(out, tensors)
        print(out, len(tensors), "tensors")
    for name in ("tiny-raw", "tiny-one", "tiny-table", "tiny-many", "tiny-reg-a", "tiny-reg-b"):
        shutil.copyfile(os.path.join(data, f"{name}.tirs"), os.path.join(HERE, f"{name}.tirs"))
        print("copied", name)
    shutil.copyfile(os.path.join(ref, "LICENSE"), os.path.join(HERE, "LICENSE-reference.txt"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
