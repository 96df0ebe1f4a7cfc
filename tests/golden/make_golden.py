#!/usr/bin/env python3
"""Writes the committed golden vectors (tests/golden/*.npz) from the CPU oracle.

Each file holds a small seeded input and the oracle's outputs for it:
  x         NCHW input in the model's input dtype
  y         oracle output, fp32 math with fp16 tensors between nodes (ONNX
            Runtime CPU EP semantics for an fp16 model)
  y_fp32    oracle output with fp32 tensors throughout (measures the fp16 floor)
The shipped-model vector uses the reference's own model and test image
(ArtCNN_R8F64_fp16.onnx and test_256.png, copied here as data fixtures).
Run from the repo root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from arthip_amd import models  # noqa: E402
from arthip_amd import onnx_proto as op  # noqa: E402
from oracle.model import run_model  # noqa: E402


def luma_crop(h: int, w: int, top: int = 64, left: int = 96) -> np.ndarray:
    """BT.601 luma of a crop of test_256.png as a 1x1xHxW fp16 frame in [0, 1]."""
    from PIL import Image
    rgb = np.asarray(Image.open(HERE / "test_256.png").convert("RGB"), np.float32) / 255.0
    y = rgb[..., 0] * 0.299 + rgb[..., 1] * 0.587 + rgb[..., 2] * 0.114
    return y[top:top + h, left:left + w][None, None].astype(np.float16)


def cases():
    yield "c4f32_24x40", models.c4f32(seed=0).model, models.synthetic_input((1, 1, 24, 40), seed=1)
    yield ("single64_12x20", models.single64(seed=0).model,
           models.synthetic_input((1, 64, 12, 20), seed=1, kind="normal"))
    yield "r8f64_20x28", models.r8f64(seed=0).model, models.synthetic_input((1, 1, 20, 28), seed=1)
    yield ("r8f64_b2_9x14", models.r8f64(seed=0).model,
           models.synthetic_input((2, 1, 9, 14), seed=2))
    yield "shipped_luma_48x64", op.load(HERE / "ArtCNN_R8F64_fp16.onnx"), luma_crop(48, 64)


def main() -> None:
    for name, model, x in cases():
        y = run_model(model, x)
        y32 = run_model(model, x, round_fp16=False)
        np.savez_compressed(HERE / f"{name}.npz", x=x, y=y, y_fp32=y32)
        print(f"{name}: x {x.shape} -> y {y.shape} range [{y.min():.3g}, {y.max():.3g}]")


if __name__ == "__main__":
    main()
