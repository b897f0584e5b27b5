"""Write the golden fixtures under tests/golden/ (run once, in the build
container where the reference checkout is mounted).

Fixtures:

* ``accuracy_gate_reference.json`` -- the reference's published accuracy-gate
  results and their exact input recipe, copied as data from its evidence
  files: shape (M, K, N) = (2048, 14336, 2048), ``default_rng(20260833)``
  uniform[-1, 1] inputs rounded to bf16, tile (2048, 2048, 512), errors vs the
  FP32 HIGHEST product
  (``archive/initial-snapshot/evidence/strassen_cubic_control.jsonl:7``,
  recipe ``experiments/qwen3/benchmark_cubic_control.py:322-336`` and
  ``experiments/qwen3/benchmark_common.py:63-69``).
* ``qwen3_0p6b_q_proj_slice.npz`` -- a [256, 512] slice (rows = output
  features, columns = input features) of the real Qwen3-0.6B layer-0 q_proj
  weight that the reference ships as test data
  (``Strassen_MM_Focus/data/qwen3-0.6b-real-v001/tensors/layer0_q_proj.bf16``,
  Apache-2.0), after checking the file's SHA-256 against the reference's
  manifest. Stored as raw bf16 bit patterns (uint16).
* ``qwen3_0p6b_down_proj_slice.npz`` -- a [256, 1024] slice (output features x
  input features) of the layer-0 down_proj weight the reference ships beside
  it (``.../tensors/layer0_down_proj.bf16``, [1024, 3072]), SHA-256 checked
  against its manifest the same way.
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = "/root/reference"
EVIDENCE = "archive/initial-snapshot/evidence/strassen_cubic_control.jsonl"
TENSOR_DIR = "Strassen_MM_Focus/data/qwen3-0.6b-real-v001/tensors"


def accuracy_gate():
    path = os.path.join(REFERENCE, EVIDENCE)
    with open(path, encoding="utf-8") as stream:
        lines = stream.read().splitlines()
    record = json.loads(lines[6])  # line 7
    assert record["kind"] == "accuracy" and record["shape"] == [2048, 14336, 2048]
    fixture = {
        "source": f"{EVIDENCE}:7",
        "shape_mkn": record["shape"],
        "seed": 20260833,
        "inputs": "numpy default_rng(seed).uniform(-1,1,(M,K)) then (K,N), float32, rounded to bf16",
        "tile_bm_bn_bk": [2048, 2048, 512],
        "tile_source": "max48 profile (strassen_pallas.py:31-35) set by benchmark_cubic_control.py:32",
        "reference": "FP32 HIGHEST matmul of the bf16 inputs",
        "errors_vs_reference": {
            name: record["errors_vs_reference"][name]
            for name in ("strassen", "cubic_blocked", "native")
        },
    }
    with open(os.path.join(HERE, "accuracy_gate_reference.json"), "w", encoding="utf-8") as stream:
        json.dump(fixture, stream, indent=1, sort_keys=True)
        stream.write("\n")


def weight_slice(name, rows, cols):
    """A [rows, cols] slice of a reference tensor, after checking the whole
    file's SHA-256 against its manifest entry."""
    meta_path = os.path.join(REFERENCE, TENSOR_DIR, f"layer0_{name}.json")
    with open(meta_path, encoding="utf-8") as stream:
        meta = json.load(stream)
    raw = open(os.path.join(REFERENCE, TENSOR_DIR, f"layer0_{name}.bf16"), "rb").read()
    digest = hashlib.sha256(raw).hexdigest()
    assert digest == meta["sha256"], f"{name} tensor does not match the reference manifest"
    full_rows, full_cols = meta["shape"]
    weight = np.frombuffer(raw, dtype="<u2").reshape(full_rows, full_cols)
    piece = np.ascontiguousarray(weight[:rows, :cols])
    np.savez(os.path.join(HERE, f"qwen3_0p6b_{name}_slice.npz"), weight_bits=piece,
             source=np.array(f"{TENSOR_DIR}/layer0_{name}.bf16[:{rows}, :{cols}]"),
             source_sha256=np.array(digest))


if __name__ == "__main__":
    accuracy_gate()
    weight_slice("q_proj", 256, 512)
    weight_slice("down_proj", 256, 1024)
    print("golden fixtures written to", HERE)
