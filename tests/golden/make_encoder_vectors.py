"""Write golden vectors for the BC4 PTQ encoder from the reference's own implementation.

The reference's endpoint search (texelator/encoder.py:35-102, driven by encode_linear_e3 at
:121-157) has no fixtures and no closed form: its integer outputs depend on torch's float32
arithmetic. This script imports that file BY PATH from the reference checkout (under a distinct
module name, so it cannot shadow this repository's package), runs it on the CPU with this
build's palette as the LUT, and stores inputs and outputs as data:

  tests/golden/encoder_vectors.npz   small cases: weight, hdiag, rows_per_chunk -> blocks, scales
  tests/golden/encoder_vectors.json  BASELINE config 1 (4096 x 4096): SHA-256 of blocks and scales

Run in the build container only (the reference does not exist on the GPU box):
    python tests/golden/make_encoder_vectors.py [/root/reference]
Generated with torch 2.10.0 (CPU).
"""
from __future__ import annotations

import hashlib
import importlib.util
import json
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import bc4  # noqa: E402
from tests.golden.cases import config1_inputs, small_cases  # noqa: E402


def load_reference_encoder(reference: Path):
    path = reference / "texelator" / "encoder.py"
    spec = importlib.util.spec_from_file_location("reference_texelator_encoder", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def encode(reference_encoder, weight: torch.Tensor, hdiag: torch.Tensor, lut: torch.Tensor, rows_per_chunk: int):
    with tempfile.TemporaryDirectory() as tmp:
        blocks_path = Path(tmp) / "w.bc4"
        scales_path = Path(tmp) / "w.scales.f32"
        reference_encoder.encode_linear_e3(weight, hdiag, lut, blocks_path, scales_path, rows_per_chunk)
        m = weight.shape[0]
        blocks = np.fromfile(blocks_path, dtype=np.uint8).reshape(m, -1)
        scales = np.fromfile(scales_path, dtype="<f4")
    return blocks, scales


def main() -> None:
    reference = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    encoder = load_reference_encoder(reference)
    lut = torch.from_numpy(bc4.palette())
    arrays = {}
    for name, (weight, hdiag, rows_per_chunk) in small_cases().items():
        blocks, scales = encode(encoder, weight, hdiag, lut, rows_per_chunk)
        arrays[f"{name}/weight"] = weight.numpy()
        arrays[f"{name}/hdiag"] = hdiag.numpy()
        arrays[f"{name}/rows_per_chunk"] = np.array(rows_per_chunk)
        arrays[f"{name}/blocks"] = blocks
        arrays[f"{name}/scales"] = scales
        print(f"{name}: {blocks.shape[0]}x{blocks.shape[1] * 2} encoded", flush=True)
    np.savez_compressed(HERE / "encoder_vectors.npz", **arrays)

    weight, hdiag = config1_inputs()
    blocks, scales = encode(encoder, weight, hdiag, lut, 128)
    record = {
        "case": "BASELINE config 1: W 4096x4096 ~ N(0, 0.02^2) * LogNormal(0, 0.3) per input channel, "
                "seed 20260827, hdiag = 1, rows_per_chunk 128",
        "torch": torch.__version__,
        "palette_sha256": bc4.palette_sha256(),
        "blocks_sha256": hashlib.sha256(blocks.tobytes()).hexdigest(),
        "scales_sha256": hashlib.sha256(scales.tobytes()).hexdigest(),
        "first_row_blocks_hex": blocks[0, :64].tobytes().hex(),
    }
    (HERE / "encoder_vectors.json").write_text(json.dumps(record, indent=2) + "\n")
    print(json.dumps(record, indent=2))


if __name__ == "__main__":
    main()
